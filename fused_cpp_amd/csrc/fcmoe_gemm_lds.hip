// fcmoe_gemm_lds.hip -- LDS-staged grouped GEMM for large row tiles
// (prefill: BM = 128 / 192 / 256 rows of one expert).
//
// Why a second kernel: at large M the MFMA pipe, not HBM, is the limit, and
// on CDNA4 every instruction that moves a 1 KB operand block through VGPRs
// (global load, LDS write, LDS read) costs MFMA issue time. This kernel
//   * stages both operands with buffer_load ... lds (global -> LDS without
//     VGPRs, issued at almost no MFMA cost),
//   * gives each wave a large 16 FM x 16 FN tile (96x128 / 128x96 / 64x128)
//     so each LDS fragment read feeds FN or FM MFMAs,
//   * keeps the accumulators in VGPRs at 2 waves per SIMD: 2 x 4 waves per
//     workgroup and one workgroup per CU, or 2 x 2 waves and two workgroups
//     per CU (the 256-row W13), whose K loops then overlap each other's
//     epilogues.
//
// Work decomposition: grid.x = tiles * n_blocks (+ spare workgroups, see
// lds_work_item); a workgroup computes rows [m0, m0 + BM) of one expert
// against WNW * FN consecutive 16-channel tiles (W13: WNW * FN/2 gate tiles
// and the matching up tiles). Waves are WMW (rows) x WNW (channel tiles).
//
// Pipeline: two LDS rings, SA stages of the A tile (BM rows) and SB >= SA
// stages of the workgroup's B tiles, one 64-byte K chunk per B stage and
// AW = 64 or 128 bytes of K per A stage. Iteration c waits for its own
// chunk-c loads (vmcnt), meets the other waves at one barrier (their chunk-c
// loads have landed; everyone is done reading chunk c-1), issues the next A
// and B stages into the ones chunk c-1 freed and computes chunk c.
//
// LDS layouts (per stage): A rows packed AW bytes apart, 16-byte unit u of
// row r at slot u ^ ((r >> 2) & 3) (AW = 64) or u ^ ((r >> 1) & 7) (AW =
// 128), so the 16 rows of a fragment read fall on distinct banks; B tiles in
// their packed MFMA operand order (1 KB per tile chunk, lane l's 16 bytes at
// 16 l). The epilogue's per-row and per-channel values follow the rings in
// the same LDS object, and the epilogue stages its output through the idle
// ring memory (staged_epilogue).
#include <cstdlib>
#include <utility>

#include "fcmoe_gemm_common.h"

namespace fcmoe {

namespace {

constexpr int kWM = 2;
constexpr int kWN = 4;
// Raw buffer resource word 3 for gfx9: 32-bit data format, no swizzle.
constexpr int kBufWord3 = 0x00020000;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(N) with the other counters unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Work order. Operand reuse across workgroups only pays when the reusing
// workgroups share an L2, and an L2 serves one XCD: L2-resident operands
// reach a CU at ~60 B/clk through buffer_load ... lds, L2 misses (Infinity
// Cache or HBM) at ~10-12 B/clk (measured on MI355X). The dispatcher deals
// workgroups to the 8 XCDs round-robin by blockIdx, so workgroup b is
// renumbered to run the (b / 8)-th item of a contiguous range of items owned
// by XCD b % 8; among the first `valid` workgroups this is a bijection, and
// at any moment each XCD runs a window of consecutive items. Items are
// ordered in groups of `gm` row tiles x all channel blocks, row tiles
// fastest: a window then holds a few row tiles against several channel
// blocks, so A (per row tile) and B (per channel block, when the row tiles
// belong to one expert) are both fetched from HBM once per window.
// gm = 0 keeps plain tile-major order.
constexpr int kXcds = 8;

// Diagnostic builds only (python -m fused_cpp_amd.build --diag N --out DIR;
// the library in the package is always built with 0). Bits: 1 skips the
// LDS-staged launches' epilogues, 2 their stage loads, 8 their fragment reads
// and MFMAs (all timing only: the results are wrong), 4 records each persistent-launch item of the W13 / W2
// epilogues (start, end of the K loop, end of the epilogue: s_memrealtime,
// 100 MHz; tile, channel block, rows, expert) into g_item_trace, read by
// fcmoe_diag_item_trace.
#ifndef FCMOE_DIAG
#define FCMOE_DIAG 0
#endif
constexpr int kDiag = FCMOE_DIAG;
constexpr int kTraceWgs = 256, kTraceItems = 64;
#if FCMOE_DIAG & 4
__device__ unsigned long long g_item_trace[2 * kTraceWgs * kTraceItems * 4];  // [W13 / W2][wg][item][4]
#endif
constexpr int kLdsGroupTiles = 4;
// gm value of a persistent launch that deals whole row tiles to the XCDs
// round-robin (see lds_work_item).
constexpr int kLdsDealTiles = 1 << 20;

// When the channel dimension does not fill the last channel block (W13 at
// F = 2048 on the 4-wave 256-row tile: 21 blocks of 6 gate/up pairs and one
// of 2), those cheaper last-block items run after all full ones, on every
// XCD: they then fill the slots left in the last round of full items instead
// of forming a round of their own (C3's 256-row W13: 3080 items on 512
// slots left 8 items, ~14% of the launch, in a seventh round). Each XCD
// takes its share of the full items, in the order above, then its share of
// the last-block items; the grid carries kXcds spare workgroups for the two
// shares' rounding.
// Row tiles dealt to XCD x (gm == kLdsDealTiles): units of kDealUnit
// consecutive tiles, unit u to XCD u % 8; the last unit may be short. Two
// tiles per unit let an XCD's L2 serve one expert's weights to both (C3:
// 3.88 GB of L2-miss traffic per W13 launch against 5.16 GB with single
// tiles, 2.77 against 2.82 ms per layer; 3 or 4 tiles per unit: 2.84 / 2.83).
constexpr int kDealUnit = 2;
__device__ __forceinline__ int deal_tiles(int count, int x) {
  constexpr int D = kDealUnit;
  const int U = (count + D - 1) / D;
  const int units_x = U / kXcds + (x < U % kXcds ? 1 : 0);
  const bool has_last = units_x > 0 && x + kXcds * (units_x - 1) == U - 1;
  return units_x * D - (has_last ? U * D - count : 0);
}

__device__ __forceinline__ bool lds_work_item(int b, int count, int n_blocks, bool partial, int gm, int& tile_idx,
                                              int& nb) {
  const int nbf = partial ? n_blocks - 1 : n_blocks;  // full channel blocks per row tile
  const int F = count * nbf, P = partial ? count : 0;
  int l, lp;
  if (gm <= 0) {
    if (b < F) {
      tile_idx = b / nbf;
      nb = b % nbf;
      return true;
    }
    lp = b - F;
  } else if (gm == kLdsDealTiles) {
    // Persistent launches only: units of kDealUnit consecutive row tiles
    // (one expert's, mostly) go to the XCDs round-robin, unit u to XCD u % 8,
    // with all their full channel blocks (row tiles fastest), then each XCD's
    // last-block items.
    const int x = b % kXcds, k = b / kXcds;
    const int tiles_x = deal_tiles(count, x);
    if (k < tiles_x * nbf) {
      constexpr int D = kDealUnit;
      const int U = (count + D - 1) / D;
      const int m = k / (D * nbf), idx = k % (D * nbf);
      const int u = x + kXcds * m;
      const int dm = u == U - 1 ? count - (U - 1) * D : D;
      tile_idx = u * D + idx % dm;
      nb = idx / dm;
      return true;
    }
    const int kp = k - tiles_x * nbf;
    if (kp >= (partial ? tiles_x : 0)) return false;
    tile_idx = (x + kXcds * (kp / kDealUnit)) * kDealUnit + kp % kDealUnit;
    nb = n_blocks - 1;
    return true;
  } else {
    const int x = b % kXcds, k = b / kXcds;
    const int qf = F / kXcds, rf = F % kXcds, qp = P / kXcds, rp = P % kXcds;
    const int nf = qf + (x < rf ? 1 : 0);
    if (k < nf) {
      l = x * qf + (x < rf ? x : rf) + k;
      const int gsz = gm * nbf;
      const int g = l / gsz, rr = l % gsz;
      const int left = count - g * gm;
      const int gm_eff = left < gm ? left : gm;
      tile_idx = g * gm + rr % gm_eff;
      nb = rr / gm_eff;
      return true;
    }
    const int kp = k - nf;
    if (kp >= qp + (x < rp ? 1 : 0)) return false;
    lp = x * qp + (x < rp ? x : rp) + kp;
  }
  if (lp >= P) return false;
  tile_idx = lp;
  nb = n_blocks - 1;
  return true;
}

// ---- staged W8A8 epilogues. The generic epilogue stores each accumulator
// value from its MFMA lane: one bf16 (W13) or one fp32 (W2) per lane and
// instruction, 16-lane pieces of four rows, plus a dword per (row, gate tile)
// for the W13 row maxima -- 192 store instructions per wave at BM = 192.
// Measured on C4 (one workgroup per CU, so nothing overlaps the epilogue),
// the W13 epilogue cost as much as 0.77 ms of a 2.4 ms launch. Here each
// wave writes a 16-row fragment into its own slice of the (now idle) stage
// memory and stores it back as row-contiguous 16-byte pieces: full cache
// lines, 8x (W13) / 4x (W2) fewer store instructions. The arithmetic is the
// generic epilogue's, value for value.
typedef __attribute__((address_space(3))) uint8_t* lds_u8_ptr;

template <int FN>
constexpr int staged_slice_bytes(int epi) {
  return epi == kEpiW13SwigluI8 ? 16 * ((FN / 2) * 32 + 16) + 16 * (FN / 2) * 4 : 16 * (FN * 64 + 16);
}

template <int EPI, int FM, int FN>
__device__ __forceinline__ void staged_epilogue(const GemmParams& p, const v4i (&acc)[FM][FN],
                                                const int64_t (&gtile)[FN], const bool (&tvalid)[FN], int row_base,
                                                int rows, int pos0, int expert, int lane, const EpiMeta& m,
                                                lds_u8_ptr slice) {
  const int col = lane % 16;
  const int rq = (lane / 16) * 4;  // first fragment row of this lane's registers
  if constexpr (EPI == kEpiW13SwigluI8) {
    constexpr int HP = FN / 2;
    constexpr int RS = HP * 32 + 16;   // bytes per staged row (HP*16 bf16 + pad: rows 4 apart on other banks)
    constexpr int UPR = HP * 2;        // 16-byte units per row
    const lds_u8_ptr rp = slice + 16 * RS;  // [16 rows][HP] row maxima
    const uint32_t ftab = fexpa_table_lane();
    float cg[HP], cu[HP];
    bool fv[HP];
#pragma unroll
    for (int j = 0; j < HP; ++j) {
      fv[j] = tvalid[j] && gtile[j] * 16 + col < p.n_half;
      cg[j] = m.cs[(m.cbase + j) * 16 + col];
      cu[j] = m.cs[(m.cbase + j + HP) * 16 + col];
    }
    const int64_t f0 = gtile[0] * 16;  // the wave's gate channels are f0 .. f0 + 16 HP - 1
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int rbase = row_base + i * 16;
      if (rbase >= rows) break;  // fragments past the expert's rows (wave-uniform)
      // Batches of QB registers x HP tiles: every table lookup of a batch is
      // issued before the first is used and the batch's 16-lane maxima run
      // side by side (one lookup and max at a time, each waited out alone,
      // made this the slowest part of the epilogue).
      constexpr int QB = 2;
#pragma unroll
      for (int q0 = 0; q0 < 4; q0 += QB) {
        float gate[QB][HP], up[QB][HP], ya[QB][HP];
        FexpaArg ea[QB][HP];
        uint32_t frac[QB][HP];
        bool rok[QB];
#pragma unroll
        for (int b = 0; b < QB; ++b) {
          const int r = rbase + rq + q0 + b;
          rok[b] = r < rows;
          const float xs = m.rs[rok[b] ? r : rows - 1];
#pragma unroll
          for (int j = 0; j < HP; ++j) {
            // w13_epilogue, csrc/moe/arm/i8mm_w8a8/kernels.cpp:230-246
            gate[b][j] = fminf((float)acc[i][j][q0 + b] * (xs * cg[j]), 10.0f);
            up[b][j] = fmaxf(fminf((float)acc[i][j + HP][q0 + b] * (xs * cu[j]), 10.0f), -10.0f);
            ea[b][j] = fexpa_reduce(gate[b][j]);
            frac[b][j] = fexpa_lookup(ea[b][j].bits, ftab);
          }
        }
#pragma unroll
        for (int b = 0; b < QB; ++b)
#pragma unroll
          for (int j = 0; j < HP; ++j) {
            const float ex = fexpa_finish(ea[b][j], frac[b][j]);
            const uint16_t yb = f32_to_bf16((gate[b][j] * up[b][j]) / (ex + 1.0f));
            *(__attribute__((address_space(3))) uint16_t*)(slice + (rq + q0 + b) * RS + (j * 16 + col) * 2) = yb;
            ya[b][j] = rok[b] && fv[j] ? fabsf(bf16_to_f32(yb)) : 0.0f;
          }
        // Row maxima over the wave's HP gate tiles at once: the lane's own
        // maximum first, then one 16-lane reduction per row. Each of the
        // row's HP partial entries gets the group maximum, which leaves the
        // maximum over all entries, the only thing the requant reads, as is.
        float ym[QB];
#pragma unroll
        for (int b = 0; b < QB; ++b) {
          ym[b] = ya[b][0];
#pragma unroll
          for (int j = 1; j < HP; ++j) ym[b] = fmaxf(ym[b], ya[b][j]);
          ym[b] = max16(ym[b]);
        }
        if (col == 0) {
#pragma unroll
          for (int b = 0; b < QB; ++b)
#pragma unroll
            for (int j = 0; j < HP; ++j)
              *(__attribute__((address_space(3))) float*)(rp + ((rq + q0 + b) * HP + j) * 4) = ym[b];
        }
      }
#pragma unroll
      for (int h = 0; h < (16 * UPR + kWave - 1) / kWave; ++h) {
        const int idx = h * kWave + lane;
        const int row = idx / UPR, u = idx % UPR;
        const int r = rbase + row;
        const int64_t ch = f0 + u * 8;
        if (idx < 16 * UPR && r < rows && ch < p.n_half) {
          const v4i v = *(__attribute__((address_space(3))) const v4i*)(slice + row * RS + u * 16);
          *(v4i*)((uint16_t*)p.out + (int64_t)(pos0 + r) * p.ldo + ch) = v;
        }
      }
      if (lane < 16 * HP) {
        const int row = lane / HP, jj = lane % HP;
        const int r = rbase + row;
        const int64_t t = gtile[0] + jj;  // the wave's gate tiles are consecutive
        if (r < rows && t < p.n_tiles)
          p.rowpart[(int64_t)(pos0 + r) * p.n_tiles + t] =
              *(__attribute__((address_space(3))) const float*)(rp + lane * 4);
      }
    }
  } else if constexpr (EPI == kEpiI8Gemm) {
    // write_scaled_output, csrc/i8gemm.cpp:148-164: (float)acc * s_x * s_w
    // left to right, + bias, then bf16 (RNE) or fp32. Staged as fp32 rows;
    // stored as 16-byte pieces of 8 bf16 or 4 fp32 channels where the row
    // stride and the channel count allow it, else channel by channel.
    constexpr int RS = FN * 64 + 16;  // bytes per staged row (FN*16 fp32 + pad)
    float cs[FN], cb[FN];
    const int64_t c0 = gtile[0] * 16;  // one channel group: the wave's channels are c0 .. c0 + 16 FN - 1
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t ch = c0 + j * 16 + col;
      cs[j] = m.cs[(m.cbase + j) * 16 + col];
      cb[j] = p.bias && tvalid[j] && ch < p.n ? p.bias[ch] : 0.0f;
    }
    // split K: this split's raw int32 sums, [split_rows, n] at split_out + split * split_rows * n
    const bool raw = p.k_total > 0;
    int32_t* const rout = raw ? p.split_out + (int64_t)blockIdx.y * p.split_rows * p.n : nullptr;
    const int per = p.out_bf16 && !raw ? 8 : 4;  // channels per 16-byte piece
    const bool vec = raw ? p.n % 4 == 0 : p.ldo % per == 0 && ((uintptr_t)p.out & 15) == 0;
    const int upr = FN * 16 / per;       // pieces per staged row
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int rbase = row_base + i * 16;
      if (rbase >= rows) break;  // fragments past the expert's rows (wave-uniform)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = rbase + rq + q;
        const float rs = m.rs[r < rows ? r : rows - 1];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float v = (float)acc[i][j][q] * rs * cs[j];
          if (p.bias) v = v + cb[j];
          *(__attribute__((address_space(3))) float*)(slice + (rq + q) * RS + (j * 16 + col) * 4) =
              raw ? __int_as_float(acc[i][j][q]) : v;
        }
      }
      for (int idx = lane; idx < 16 * upr; idx += kWave) {
        const int row = idx / upr, u = idx % upr;
        const int r = rbase + row;
        const int64_t ch = c0 + (int64_t)u * per;
        if (r >= rows || ch >= p.n) continue;
        const int64_t o = (int64_t)(pos0 + r) * (raw ? p.n : p.ldo) + ch;
        const __attribute__((address_space(3))) float* src =
            (const __attribute__((address_space(3))) float*)(slice + row * RS + u * per * 4);
        if (raw) {
          if (vec && ch + per <= p.n) {
            *(v4i*)(rout + o) = *(const __attribute__((address_space(3))) v4i*)src;
          } else {
            for (int e = 0; e < per && ch + e < p.n; ++e) rout[o + e] = __float_as_int(src[e]);
          }
        } else if (vec && ch + per <= p.n) {
          if (p.out_bf16) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              w[e] = (uint32_t)f32_to_bf16(src[2 * e]) | ((uint32_t)f32_to_bf16(src[2 * e + 1]) << 16);
            *(v4i*)((uint16_t*)p.out + o) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
          } else {
            *(v4i*)((float*)p.out + o) = *(const __attribute__((address_space(3))) v4i*)src;
          }
        } else {
          for (int e = 0; e < per && ch + e < p.n; ++e) {
            if (p.out_bf16)
              ((uint16_t*)p.out)[o + e] = f32_to_bf16(src[e]);
            else
              ((float*)p.out)[o + e] = src[e];
          }
        }
      }
    }
  } else {  // kEpiW2RouteI8: store_w2, csrc/moe/arm/i8mm_w8a8/kernels.cpp:248-257
    constexpr int RS = FN * 64 + 16;  // bytes per staged row (FN*16 fp32 + pad)
    constexpr int UPR = FN * 4;       // 16-byte units per row
    float cs[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) cs[j] = m.cs[(m.cbase + j) * 16 + col];
    const int64_t c0 = gtile[0] * 16;  // the wave's channels are c0 .. c0 + 16 FN - 1
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int rbase = row_base + i * 16;
      if (rbase >= rows) break;  // fragments past the expert's rows (wave-uniform)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = rbase + rq + q;
        const float rs = m.rs[r < rows ? r : rows - 1];
#pragma unroll
        for (int j = 0; j < FN; ++j)
          *(__attribute__((address_space(3))) float*)(slice + (rq + q) * RS + (j * 16 + col) * 4) =
              (float)acc[i][j][q] * (rs * cs[j]);
      }
#pragma unroll
      for (int h = 0; h < 16 * UPR / kWave; ++h) {
        const int idx = h * kWave + lane;
        const int row = idx / UPR, u = idx % UPR;
        const int r = rbase + row;
        const int64_t ch = c0 + u * 4;
        if (r < rows && ch < p.n) {
          const int orow = m.orow[r];
          const v4i v = *(__attribute__((address_space(3))) const v4i*)(slice + row * RS + u * 16);
          // nontemporal: the route rows are read once, by the combine after
          // the whole launch, long after any cache would have kept them (C3
          // 2.76 -> 2.73 ms, C4 4.60 -> 4.55 ms, the combine included)
          __builtin_nontemporal_store(v, (v4i*)((float*)p.out + (int64_t)orow * p.ldo + ch));
        }
      }
    }
  }
  (void)expert;
}

template <bool I8, int EPI, int FM, int FN, int SA, int SB, int BPOL, int AW, int WMW, int WNW, bool PERSIST>
__device__ __forceinline__ void lds_gemm_body(const GemmParams& p, int n_blocks, int partial, int gm, int grid_items) {
  // The body is device-only: the buffer-resource type does not exist for the
  // host target, and the host pass needs only the kernel's signature.
#if __HIP_DEVICE_COMPILE__
  constexpr int WAVES = WMW * WNW;
  constexpr int THREADS = WAVES * kWave;
  constexpr int BM = WMW * FM * 16;
  constexpr int NT = WNW * FN;            // channel tiles per workgroup
  // AW = 128: each A stage holds two K chunks (128 bytes of every row) and
  // is loaded as full 128-byte lines, 8 rows per load. A half-line load (16
  // rows x 64 bytes) costs the CU's L1 one L2 request per 64 bytes; the
  // number of requests a CU keeps in flight, not HBM or L2 bandwidth, bounded
  // the A+B intake (~12 B/clk per CU at 80% L2 hits, L1 pending-stalled 33%
  // of the time).
  static_assert(AW == 64 || AW == 128, "A stage K width");
  constexpr bool AWIDE = AW == 128;
  // W8A16: bf16 A rows against int8 weight tiles. A K chunk is 64 elements:
  // one 128-byte A stage (the AW = 128 layout) per 1 KB weight-tile chunk,
  // and each chunk runs two bf16 MFMAs per (row fragment, tile) on the
  // widened weights. With int8 A, an AW = 128 stage holds two chunks.
  constexpr bool W8 = epi_w8(EPI);
  static_assert(!W8 || (!I8 && AWIDE), "W8A16 tiles stage 128-byte bf16 A chunks");
  constexpr bool APAIR = AWIDE && !W8;  // one A stage holds two K chunks
  constexpr int A_BYTES = BM * AW;        // one A stage
  constexpr int B_BYTES = NT * 1024;      // one B stage
  constexpr int LA = BM * AW / 1024;      // A loads (1 KB each) per stage
  constexpr int LB = NT;                  // B loads (one 1 KB tile chunk) per chunk
  constexpr int LPA = (LA + WAVES - 1) / WAVES;  // per wave
  constexpr int LPB = (LB + WAVES - 1) / WAVES;
  // vector-memory ops a wave may still have in flight once chunk c's A and B
  // have landed (see the issue order below)
  // (B c precedes A c when SB > SA; with SB == SA it is A c's pair partner)
  constexpr int WAIT_A = LPB + (SA - 2) * (LPA + LPB);
  constexpr int WAIT_B = (SB - 2) * (LPA + LPB);
  constexpr int WAIT = WAIT_A < WAIT_B ? WAIT_A : WAIT_B;
  // AW = 128 (SA = 2 stages of two chunks, SB = 3): even iterations wait for
  // A c/2 and B c, odd ones for B c (see the loop)
  constexpr int WAIT_EVEN = LPB;
  constexpr int WAIT_ODD = LPA + LPB;
  static_assert(!APAIR || (SA == 2 && SB == 3), "paired A stages run 2 A stages and 3 B stages");
  constexpr bool PAIR = epi_pair(EPI);
  constexpr int HP = FN / 2;
  static_assert(SA >= 2 && SB >= SA, "A ring of 2+ stages, B ring at least as deep");
  static_assert(WAIT < 64, "vmcnt range");
  static_assert(SA * A_BYTES + SB * B_BYTES + 8 * BM + 64 * NT + 16 <= 160 * 1024, "LDS budget");
  static_assert(NT * 16 <= THREADS && BM <= THREADS, "one metadata value per thread");
  static_assert(FM >= 3, "the fragment ring runs two fragments ahead");
  typedef typename Acc<I8>::type AccT;

  // One LDS object: the stage rings, then the epilogue metadata. (With a
  // second __shared__ object the compiler could no longer tell the fragment
  // reads apart from the in-flight buffer_load ... lds writes and put a
  // vmcnt(0) in every K iteration, draining the prefetch ring.)
  constexpr int META = SA * A_BYTES + SB * B_BYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[META + 8 * BM + 64 * NT + 16];
  float* const meta_rs = (float*)(smem + META);
  int* const meta_orow = (int*)(smem + META + 4 * BM);
  float* const meta_cs = (float*)(smem + META + 8 * BM);
  uint8_t* const smem_b = smem + SA * A_BYTES;

  // A persistent launch whose plan is not taken may still run the 256-row
  // class of the partitioned classic plan on its first part_wgs workgroups.
  bool part = false;
  if (!plan_open(p)) {
    if (!PERSIST || !p.part_counts || (int)blockIdx.x >= part_wgs(p.part_counts)) return;
    part = true;
  }
  if (part && gm == kLdsDealTiles) gm = kLdsGroupTiles;  // the partitioned plan keeps XCD windows
  const int32_t* const tiles0 = part ? p.part_tiles : p.tiles;
  int32_t* const queue = part ? p.part_queue : p.queue;
  const int u_n = part ? 0 : p.u_n;
  // Item space: one class's tile list, or (u_n > 0) several lists back to back.
  int ucount[3] = {0, 0, 0};
  int count;
  if constexpr (PERSIST) {
    count = 0;
    for (int u = 0; u < u_n; ++u) {
      ucount[u] = *p.u_count[u];
      count += ucount[u];
    }
    if (u_n == 0) count = part ? p.part_counts[3] : *p.tile_count;
  } else {
    count = *p.tile_count;
  }
  // Persistent launches (p.persist > 0): gridDim.x workgroups (a multiple of
  // the XCD count, so an item keeps its XCD) loop over the item slots of
  // their XCD, x + 8 k: with a queue, k comes from the XCD's counter (the
  // next item, whatever the other workgroups' items cost); without one,
  // workgroup b takes k = b / 8, b / 8 + gridDim.x / 8, ... Otherwise each
  // workgroup runs slot blockIdx.x.
  // (in the one LDS object: a second __shared__ object costs the K loop a
  // vmcnt(0) per chunk, see above)
  int* const next_k = (int*)(smem + META + 8 * BM + 64 * NT);
  const int xcd = (int)blockIdx.x % kXcds;
  int xcd_items = 0;  // valid slots of this XCD (lds_work_item's layout)
  if constexpr (PERSIST) {
    const int nbf = partial ? n_blocks - 1 : n_blocks;
    const int F = count * nbf, P = partial ? count : 0;
    xcd_items = F / kXcds + (xcd < F % kXcds ? 1 : 0) + P / kXcds + (xcd < P % kXcds ? 1 : 0);
    if (gm == kLdsDealTiles) xcd_items = deal_tiles(count, xcd) * (nbf + (partial ? 1 : 0));
    if (gm <= 0) xcd_items = grid_items;  // plain order: slots are not XCD-local
  }
  auto fetch_k = [&](int k_static) -> int {
    if (!PERSIST || !queue) return k_static;
    __syncthreads();  // everyone has read the previous next_k
    if (threadIdx.x == 0) *next_k = __hip_atomic_fetch_add(queue + xcd, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return *next_k;
  };
  int k = PERSIST ? fetch_k((int)blockIdx.x / kXcds) : 0;
  for (int it = 0, slot = (int)blockIdx.x; PERSIST ? k < xcd_items : it < 1; ++it) {
  if constexpr (PERSIST) slot = gm <= 0 ? (int)blockIdx.x + it * (int)gridDim.x : k * kXcds + xcd;
  int tile_idx, nb;
  const bool have = lds_work_item(slot, count, n_blocks, partial != 0, gm, tile_idx, nb);
  if constexpr (PERSIST) {
    k = fetch_k(k + (int)gridDim.x / kXcds);
    if (gm <= 0) k = slot + (int)gridDim.x < grid_items ? 0 : xcd_items;  // plain order: stride over all slots
    if (!have) continue;
    if (it > 0) __syncthreads();  // the previous item's epilogue is done with the stages
  } else {
    if (!have) return;
  }
  // last-first within a list, as the register kernel
  const int32_t* tpair = tiles0 + 2 * (count - 1 - tile_idx);
  if constexpr (PERSIST) {
    if (u_n > 0) {
      int t = tile_idx, u = 0;
      while (u + 1 < u_n && t >= ucount[u]) t -= ucount[u++];
      tpair = p.u_tiles[u] + 2 * (ucount[u] - 1 - t);
    }
  }
  const int expert = tpair[0];
  const int m0 = tpair[1];
  const int rows_left = p.counts[expert] - m0;
  const int rows = rows_left < BM ? rows_left : BM;
  const int pos0 = p.offsets[expert] + m0;
#if FCMOE_DIAG & 4
  unsigned long long* const trp =
      PERSIST && (EPI == kEpiW13SwigluI8 || EPI == kEpiW2RouteI8) && blockIdx.x < kTraceWgs && it < kTraceItems &&
              threadIdx.x == 0
          ? g_item_trace + (((EPI == kEpiW2RouteI8 ? kTraceWgs : 0) + blockIdx.x) * kTraceItems + it) * 4
          : nullptr;
  if (trp) {
    trp[0] = __builtin_amdgcn_s_memrealtime();
    trp[3] = (unsigned long long)tile_idx | ((unsigned long long)nb << 16) | ((unsigned long long)rows << 32) |
             ((unsigned long long)expert << 48);
  }
#endif

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = wave / WNW;
  const int wn = wave % WNW;
  // K range: all k_chunks chunks, or (split K, k_total > 0) split blockIdx.y's
  // range of k_chunks chunks out of k_total (the host sizes the splits so
  // that every range is non-empty and, with two-chunk A stages, starts even)
  // (compiled for the i8gemm epilogue only: the other tiles' register
  // budgets have no room for it)
  constexpr bool SPLIT = EPI == kEpiI8Gemm && !PERSIST;
  const int64_t ktot = SPLIT && p.k_total > 0 ? p.k_total : p.k_chunks;
  const int64_t kbeg = SPLIT && p.k_total > 0 ? (int64_t)blockIdx.y * p.k_chunks : 0;
  const int64_t kc = p.k_chunks < ktot - kbeg ? p.k_chunks : ktot - kbeg;
  const int64_t total_tiles = (int64_t)p.n_groups * p.n_tiles;

  // channel tile (index within the expert) of wave column wn_, slot j
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

  // ---- buffer resources and this wave's loads per stage: A loads g = wave,
  // wave + WAVES, ... (1 KB each: 16 rows x 64 bytes, or 8 rows x 128
  // bytes), B loads likewise over the NT tiles; indices past the count repeat
  // an earlier load (same bytes to the same place) so every wave issues
  // exactly LPA + LPB loads.
  const int64_t lda_bytes = p.lda * (I8 ? 1 : 2);
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.a), (short)0, 0x7ffffff0, kBufWord3);
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.w + (int64_t)expert * p.w_expert_bytes), (short)0,
      (int)(p.w_expert_bytes < 0x7ffffff0 ? p.w_expert_bytes : 0x7ffffff0), kBufWord3);
  uint32_t voff_a[LPA], voff_b[LPB];
  int lds_a[LPA], lds_b[LPB];
#pragma unroll
  for (int u = 0; u < LPA; ++u) {
    int g = wave + WAVES * u;
    while (g >= LA) g -= LA;
    // AW = 64: rows 16 g + lane / 4, 16-byte unit (lane % 4) stored at slot
    // unit ^ ((r >> 2) & 3). AW = 128: rows 8 g + lane / 8, unit u of row r
    // stored at slot u ^ ((r >> 1) & 7). Either way the 16 rows of a
    // fragment read fall on distinct banks.
    const int r = AWIDE ? g * 8 + lane / 8 : g * 16 + lane / 4;
    const int unit = AWIDE ? (lane % 8) ^ ((r >> 1) & 7) : (lane % 4) ^ ((lane >> 4) & 3);
    const int pos = pos0 + (r < rows ? r : rows - 1);
    const int64_t arow = p.row_map ? (int64_t)p.row_map[pos] : (int64_t)pos;
    // Rows past the tile's rows load from past the buffer resource's range
    // (num_records 0x7ffffff0; 0x80000040, and 0x80000000 after the fold's
    // -64 below, stay past it, as does either plus a K offset < 2^31): the
    // load still counts in vmcnt (every wave's wait counts stay uniform) but
    // moves no data, and the stage gets zeros there, which no epilogue
    // stores. (They used to re-read the last row: L2 hits, but intake of a CU
    // whose vector-memory path the stage loads share.)
    voff_a[u] = r < rows ? (uint32_t)(arow * lda_bytes + unit * 16) : 0x80000040u;
    lds_a[u] = g * 1024;
  }
  // B: a load's tile is the same for the whole wave, so its offset goes in
  // the scalar operand and every B load shares one lane offset register.
  const uint32_t voff_lane = (uint32_t)lane * 16;
#pragma unroll
  for (int u = 0; u < LPB; ++u) {
    int t = wave + WAVES * u;
    while (t >= LB) t -= LB;
    bool valid;
    const int64_t gt = tile_of(t / FN, t % FN, &valid);
    voff_b[u] = (uint32_t)__builtin_amdgcn_readfirstlane((int)((valid ? gt : 0) * ktot * 1024));
    lds_b[u] = t * 1024;
  }
  // Past the end a ring re-loads the last chunk (never read).
  // AW = 128: c counts stages (pairs of chunks). With an odd chunk count the
  // last stage's second half lies past K (past the buffer for the last A
  // row): its lanes re-load the first half instead (never read).
  const int64_t a_stages = APAIR ? (kc + 1) / 2 : kc;
  const bool a_hi = AWIDE && ((lane % 8) ^ ((((wave & 1) << 2) | (lane >> 4)) & 7)) >= 4;
  auto issue_a = [&](int64_t c, int stage) {
    if constexpr (kDiag & 2) return;
    const int64_t cc = c < a_stages ? c : a_stages - 1;
    const int soff = (int)(kbeg * 64 + cc * AW);
    const bool fold = APAIR && kbeg + 2 * cc + 1 >= ktot;
#pragma unroll
    for (int u = 0; u < LPA; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_ptr_t)(smem + stage * A_BYTES + lds_a[u]), 16,
                                               fold && a_hi ? voff_a[u] - 64 : voff_a[u], soff, 0, 0);
  };
  auto issue_b = [&](int64_t c, int stage) {
    if constexpr (kDiag & 2) return;
    const int soff = (int)((kbeg + (c < kc ? c : kc - 1)) * 1024);
#pragma unroll
    for (int u = 0; u < LPB; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b, (lds_ptr_t)(smem_b + stage * B_BYTES + lds_b[u]), 16,
                                               voff_lane, (int)voff_b[u] + soff, 0, BPOL);
  };

  // A wave whose channel tiles all lie past the end (the last channel block
  // of a launch whose channels do not fill it) skips its MFMAs; it still
  // issues its share of the loads and meets every barrier. Compiled for the
  // 6-tile waves only (the 256-row tiles, whose blocks do not divide the
  // DeepSeek channel counts); elsewhere the branch cost the 192-row tile a
  // register spill and its blocks divide evenly.
  bool wave_live = FN != 6;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    bool v;
    (void)tile_of(wn, j, &v);
    wave_live = wave_live || v;
  }
  // Persistent launches also take experts of fewer rows than the tile: a
  // wave whose row fragments all lie past the expert's rows skips its MFMAs.
  if constexpr (PERSIST) wave_live = wave_live && wm * FM * 16 < rows;
  // row fragments of this wave that hold rows of the expert (the rest are clamped re-reads of its last row)
  const int live_frags = __builtin_amdgcn_readfirstlane((rows - wm * FM * 16 + 15) / 16);

  // ---- fragment addresses (bytes within a stage)
  constexpr int A_FRAG = 16 * AW;  // bytes per 16-row fragment in a stage
  // W8A16 reads units 2 g and 2 g + 1 (g = lane / 16) of its row: slots
  // (2 g) ^ x and ((2 g) ^ x) ^ 1, i.e. a_frag and a_frag + a_dhi.
  const int a_unit = W8 ? 2 * (lane / 16) : lane / 16;
  const int a_frag = AWIDE ? (wm * FM * 16 + lane % 16) * 128 + ((a_unit ^ ((lane % 16) >> 1)) * 16)
                           : (wm * FM * 16 + lane % 16) * 64 + (((lane / 16) ^ ((lane % 16) >> 2)) * 16);
  const int a_dhi = (a_frag ^ 16) - a_frag;

  const int b_frag = wn * FN * 1024 + lane * 16;

  AccT acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = AccT{0, 0, 0, 0};

  // ---- epilogue metadata, phase 1: per-row (thread t < BM: row t) and
  // per-channel (thread t: slot t / 16, column t % 16) values into registers.
  // Their round trip coincides with the row_map loads the A offsets above
  // already wait for; phase 2 follows the prologue.
  constexpr bool ROUTE = epi_route(EPI);
  constexpr bool COLS = epi_col_scale(EPI);
  const int mt = threadIdx.x;
  int m_row = 0, m_orow = 0;
  float m_rs = 0.0f, m_cs = 0.0f;
  if (mt < BM) {
    const int pos = pos0 + (mt < rows ? mt : rows - 1);
    if constexpr (EPI == kEpiW13SwigluI8) m_row = p.row_map ? p.row_map[pos] : pos;
    if constexpr (EPI == kEpiW2RouteI8 || EPI == kEpiI8Gemm) m_rs = p.scale_row[pos];
    m_orow = ROUTE ? p.sorted_routes[pos] : pos;
  }
  if constexpr (COLS) {
    if (mt < NT * 16) {
      bool valid;
      const int64_t gt = tile_of(mt / 16 / FN, (mt / 16) % FN, &valid);
      const int64_t g = gt / p.n_tiles;
      const int64_t cin = (gt - g * p.n_tiles) * 16 + mt % 16;
      if (valid && cin < p.n_half)
        m_cs = p.scale_col[(EPI == kEpiI8Gemm ? 0 : (int64_t)expert * p.n) + g * p.n_half + cin];
    }
  }

  // Issue order (AW = 64): B chunks 0 .. SB-SA-1 alone, then pairs
  // (A m, B m+SB-SA), one pair per iteration after the prologue. When
  // iteration c waits, the ops issued after A c are B c+SB-SA and the SA-2
  // later pairs: WAIT. B runs SB-SA chunks further ahead than A: the weights
  // stream from HBM (long latency), A rows are re-read from L2.
  // AW = 128: A stage 0, B 0, B 1; then even iteration c issues A stage
  // c/2 + 1 and B c+2, odd iteration c issues B c+2.
  if constexpr (APAIR) {
    issue_a(0, 0);
    issue_b(0, 0);
    issue_b(1, 1);
  } else {
#pragma unroll
    for (int s = 0; s < SB - SA; ++s) issue_b(s, s);
#pragma unroll
    for (int s = 0; s < SA - 1; ++s) {
      issue_a(s, s);
      issue_b(s + SB - SA, s + SB - SA);
    }
  }
  // ---- epilogue metadata, phase 2: the W13 row scale (indexed by the row's
  // token) and the LDS writes; the K loop's first barrier publishes them.
  if (mt < BM) {
    if constexpr (EPI == kEpiW13SwigluI8) m_rs = p.scale_row[m_row];
    meta_rs[mt] = m_rs;
    meta_orow[mt] = m_orow;
  }
  if constexpr (COLS) {
    if (mt < NT * 16) meta_cs[mt] = m_cs;
  }
  // Retire the scalar loads of the set-up here: with one still pending at the
  // loop header the first fragment wait of every chunk becomes lgkmcnt(0).
  __builtin_amdgcn_s_waitcnt(0xC07F);
  // One chunk: fragment reads in consumption order (A row 0, the B tiles, A
  // row 1), then one A read two rows ahead per row of MFMAs. The schedule is
  // pinned: left to itself the compiler sinks each read next to its first use
  // and every row then waits out the LDS latency.
  auto compute = [&](const uint8_t* sta, const uint8_t* stb) {
    if constexpr (kDiag & 8) return;
    v4i bf[FN];
    v4i af[3];
    af[0] = *(const v4i*)(sta);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *(const v4i*)(stb + b_frag + j * 1024);
    af[1] = *(const v4i*)(sta + A_FRAG);
    __builtin_amdgcn_sched_group_barrier(0x100, FN + 2, 0);  // the FN + 2 leading LDS reads
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (i + 2 < FM) af[(i + 2) % 3] = *(const v4i*)(sta + (i + 2) * A_FRAG);
      // persistent launches: row fragments past the expert's rows skip their MFMAs
      if (PERSIST && i >= live_frags) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (I8) {
          acc[i][j] = mfma(af[i % 3], bf[j], acc[i][j]);
        } else {
          acc[i][j] = mfma(__builtin_bit_cast(v8bf, af[i % 3]), __builtin_bit_cast(v8bf, bf[j]), acc[i][j]);
        }
      }
      if (i + 2 < FM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // A read for row i + 2
      __builtin_amdgcn_sched_group_barrier(0x008, FN, 0);                 // then row i's MFMAs
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // W8A16 chunk. Lane l's weight bytes are K 16 g .. 16 g + 15 of its column
  // (g = l / 16); widened, they pair with A units 2 g and 2 g + 1 of its row
  // (K 16 g .. 16 g + 7 and 16 g + 8 .. 16 g + 15), which sit in adjacent
  // slots of the swizzled stage (slot (2 g) ^ x and that slot ^ 1). The
  // weights are widened once per chunk and reused by every row fragment.
  auto compute_w8 = [&](const uint8_t* sta, const uint8_t* stb) {
    if constexpr (W8) {
    v4i bl[FN], bh[FN];
    v4i af[2][2];
    {
      v4i braw[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) braw[j] = *(const v4i*)(stb + b_frag + j * 1024);
      af[0][0] = *(const v4i*)(sta);
      af[0][1] = *(const v4i*)(sta + a_dhi);
      __builtin_amdgcn_sched_group_barrier(0x100, FN + 2, 0);  // the leading LDS reads
#pragma unroll
      for (int j = 0; j < FN; ++j) i8x16_to_bf16(braw[j], bl[j], bh[j]);
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (i + 1 < FM) {
        af[(i + 1) % 2][0] = *(const v4i*)(sta + (i + 1) * A_FRAG);
        af[(i + 1) % 2][1] = *(const v4i*)(sta + (i + 1) * A_FRAG + a_dhi);
      }
      // row fragments past the expert's rows skip their MFMAs (an expert
      // of 33-64 rows fills half of the 128-row tile)
      if (i >= live_frags) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        acc[i][j] = mfma(__builtin_bit_cast(v8bf, af[i % 2][0]), __builtin_bit_cast(v8bf, bl[j]), acc[i][j]);
        acc[i][j] = mfma(__builtin_bit_cast(v8bf, af[i % 2][1]), __builtin_bit_cast(v8bf, bh[j]), acc[i][j]);
      }
      if (i + 1 < FM) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // A reads for row i + 1
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * FN, 0);             // then row i's MFMAs
    }
    __builtin_amdgcn_sched_barrier(0);
    }
  };
  if constexpr (APAIR) {
    int sa = 0, sb = 0;
    for (int64_t c = 0; c < kc; c += 2) {
      wait_vmcnt<WAIT_EVEN>();  // A stage c/2 and B c have landed
      __builtin_amdgcn_s_barrier();
      // everyone is done with chunk c-1: A stage c/2-1 and B stage c-1 are free
      issue_a(c / 2 + 1, sa ^ 1);
      issue_b(c + 2, sb == 0 ? 2 : sb - 1);
      if (wave_live) compute(smem + sa * A_BYTES + a_frag, smem_b + sb * B_BYTES);
      sb = sb == 2 ? 0 : sb + 1;
      if (c + 1 < kc) {
        wait_vmcnt<WAIT_ODD>();  // B c+1 has landed
        __builtin_amdgcn_s_barrier();
        issue_b(c + 3, sb == 0 ? 2 : sb - 1);
        // second chunk of the stage: units 4..7, i.e. slot bit 2 flipped ((4 | u) ^ x == (u ^ x) ^ 4)
        if (wave_live) compute(smem + sa * A_BYTES + (a_frag ^ 64), smem_b + sb * B_BYTES);
        sb = sb == 2 ? 0 : sb + 1;
      }
      sa ^= 1;
    }
  } else {
    int sa = 0, sb = 0;
    for (int64_t c = 0; c < kc; ++c) {
      wait_vmcnt<WAIT>();  // this wave's chunk-c A and B have landed
      __builtin_amdgcn_s_barrier();
      // everyone is done with chunk c-1: its stages take the next chunks
      issue_a(c + SA - 1, sa == 0 ? SA - 1 : sa - 1);
      issue_b(c + SB - 1, sb == 0 ? SB - 1 : sb - 1);
      if (wave_live) {
        if constexpr (W8)
          compute_w8(smem + sa * A_BYTES + a_frag, smem_b + sb * B_BYTES);
        else
          compute(smem + sa * A_BYTES + a_frag, smem_b + sb * B_BYTES);
      }
      sa = sa == SA - 1 ? 0 : sa + 1;
      sb = sb == SB - 1 ? 0 : sb + 1;
    }
  }
  wait_vmcnt<0>();  // the trailing (unused) stage loads
#if FCMOE_DIAG & 4
  if (trp) trp[1] = __builtin_amdgcn_s_memrealtime();
#endif

  int64_t gtile[FN];
  bool tvalid[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) gtile[j] = tile_of(wn, j, &tvalid[j]);
  const EpiMeta meta{(lds_cfloat_ptr)meta_rs, (lds_cint_ptr)meta_orow, (lds_cfloat_ptr)meta_cs, wn * FN};
  if constexpr (EPI == kEpiW13SwigluI8 || EPI == kEpiW2RouteI8 || EPI == kEpiI8Gemm) {
    static_assert(WAVES * staged_slice_bytes<FN>(EPI) <= SA * A_BYTES + SB * B_BYTES, "staging slices fit the stages");
    // every wave is past its last chunk's fragment reads: the stages are free
    __builtin_amdgcn_s_barrier();
    if constexpr (!(kDiag & 1))
      staged_epilogue<EPI, FM, FN>(p, acc, gtile, tvalid, wm * FM * 16, rows, pos0, expert, lane, meta,
                                   (lds_u8_ptr)(smem + wave * staged_slice_bytes<FN>(EPI)));
  } else {
    if constexpr (!(kDiag & 1))
      gemm_epilogue<I8, EPI, FM, FN, true>(p, acc, gtile, tvalid, wm * FM * 16, rows, pos0, expert, lane, meta);
  }
  if constexpr (kDiag & 1) {
    // no epilogue: every accumulator is still consumed (an empty asm
    // statement), so the fragment reads and MFMAs stay
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) asm volatile("" ::"v"(acc[i][j]));
  }
#if FCMOE_DIAG & 4
  if (trp) trp[2] = __builtin_amdgcn_s_memrealtime();
#endif
  }
#endif
}

template <bool I8, int EPI, int FM, int FN, int SA, int SB, int BPOL, int AW, int WMW, int WNW>
__global__ __launch_bounds__(WMW * WNW * kWave) void grouped_gemm_lds_kernel(GemmParams p, int n_blocks, int partial,
                                                                            int gm, int grid_items) {
  lds_gemm_body<I8, EPI, FM, FN, SA, SB, BPOL, AW, WMW, WNW, false>(p, n_blocks, partial, gm, grid_items);
}

// Persistent form: gridDim.x workgroups loop over the items.
template <bool I8, int EPI, int FM, int FN, int SA, int SB, int BPOL, int AW, int WMW, int WNW>
__global__ __launch_bounds__(WMW * WNW * kWave) void
grouped_gemm_lds_persist_kernel(GemmParams p, int n_blocks, int partial, int gm, int grid_items) {
  lds_gemm_body<I8, EPI, FM, FN, SA, SB, BPOL, AW, WMW, WNW, true>(p, n_blocks, partial, gm, grid_items);
}

// Channel blocks per row tile of a workgroup whose waves hold FN 16-channel
// tiles (W13: FN/2 gate/up pairs).
template <int EPI>
int64_t lds_blocks(int wn, int fn, const GemmParams& p) {
  constexpr bool PAIR = epi_pair(EPI);
  const int64_t per_block = PAIR ? (int64_t)wn * (fn / 2) : (int64_t)wn * fn;
  const int64_t units = PAIR ? p.n_tiles : (int64_t)p.n_groups * p.n_tiles;
  return ceil_div(units, per_block);
}

template <bool I8, int EPI, int FM, int FN, int SA, int SB, int BPOL, int AW, int WMW = kWM, int WNW = kWN,
          bool PERSIST = false>
int launch_lds_cfg(const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  const int64_t n_blocks = lds_blocks<EPI>(WNW, FN, p);
  if (max_tiles * n_blocks <= 0) return FCMOE_OK;
  constexpr bool PAIR = epi_pair(EPI);
  const int64_t units = PAIR ? p.n_tiles : (int64_t)p.n_groups * p.n_tiles;
  const int partial = n_blocks * (PAIR ? WNW * (FN / 2) : WNW * FN) > units ? 1 : 0;
  const int64_t items = max_tiles * n_blocks + (partial ? kXcds : 0);
  if (items > INT32_MAX) return fail(FCMOE_EINVAL, "grouped gemm grid too large");
  const int64_t grid = PERSIST && items > p.persist ? p.persist : items;
  // split K (non-persistent launches only): one grid row per K range
  const int64_t splits = !PERSIST && p.k_total > 0 ? ceil_div(p.k_total, p.k_chunks) : 1;
  if (splits > 65535) return fail(FCMOE_EINVAL, "grouped gemm: too many K splits");
  // 32-bit buffer offsets: A rows and one expert's packed weights
  if (p.w_expert_bytes >= 0x7ffffff0) return fail(FCMOE_EINVAL, "expert weights exceed 2 GiB");
  static const int gm = [] {
    const char* v = getenv("FCMOE_LDS_GROUP");
    return v ? atoi(v) : kLdsGroupTiles;
  }();
  // The mixed plan's launches deal row tiles to the XCDs round-robin
  // (kLdsDealTiles) instead of contiguous ranges: their item space runs from
  // full 256-row tiles down to the cheaper partial and 128-row ones, and
  // contiguous ranges left the XCDs holding the cheap end idle while others
  // still ran (C3 2.89 -> 2.77 ms per layer, T = 8192 5.00 -> 4.67 ms). The
  // partitioned plan's launch keeps the 4-tile windows (no better dealt).
  const int gm_launch = PERSIST && p.u_n > 0 ? kLdsDealTiles : gm;
  if constexpr (PERSIST)
    hipLaunchKernelGGL((grouped_gemm_lds_persist_kernel<I8, EPI, FM, FN, SA, SB, BPOL, AW, WMW, WNW>),
                       dim3((unsigned)grid), dim3(WMW * WNW * kWave), 0, stream, p, (int)n_blocks, partial,
                       gm_launch, (int)items);
  else
    hipLaunchKernelGGL((grouped_gemm_lds_kernel<I8, EPI, FM, FN, SA, SB, BPOL, AW, WMW, WNW>),
                       dim3((unsigned)grid, (unsigned)splits), dim3(WMW * WNW * kWave), 0, stream, p, (int)n_blocks,
                       partial, gm, (int)items);
  return check_launch("grouped_gemm_lds");
}

template <bool I8, int EPI>
int launch_lds_bm(int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  // Weight stages of the 128/192-row classes load nontemporal: an expert in
  // those classes has one row tile, so its weights are read exactly once and
  // caching them only evicts the A rows the other channel blocks re-read.
  // The 256-row class holds every larger expert, whose row tiles re-read the
  // same weights, which stay cached (C4: W13 bm192 2.48 -> 2.40 ms; C3's
  // W2 bm256 0.63 -> 0.66 ms with nontemporal weights).
  constexpr int kNT = 2;  // buffer-load cache policy bit: nontemporal
  // A stages are 128 bytes of K (two chunks, full-line loads) where the
  // register budget allows it.
  switch (bm) {
    case 128:
      return launch_lds_cfg<I8, EPI, 4, 8, 2, 3, kNT, 128>(p, max_tiles, stream);
    case 192:
      // 128-byte A stages cut C4's W13 bm192 (streaming 11.3 GB of weights)
      // from 2.33 to 2.10 ms: fewer L2 requests per A byte leave more of the
      // CU's outstanding-request budget to the weight stream. The bf16
      // epilogues would spill with them and keep 64-byte A stages.
      if constexpr (EPI == kEpiI8Gemm)  // i8gemm takes 256-row tiles above the small-M kernel's rows
        return fail(FCMOE_EINVAL, "i8gemm has no 192-row tile");
      else if constexpr (I8)
        return launch_lds_cfg<I8, EPI, 6, 8, 2, 3, kNT, 128>(p, max_tiles, stream);
      else
        return launch_lds_cfg<I8, EPI, 6, 8, 3, 3, kNT, 64>(p, max_tiles, stream);
    case 256:
      // The mixed plan's persistent launch: 2 x 4 waves of 128 x 64 (at most
      // 216 VGPRs, 115 KB of LDS), so that the 16-row streaming launch's
      // waves (64 VGPRs) fit on every SIMD beside two of its waves.
      // (not for the raw-sum diagnostic, which never runs persistent)
      if constexpr (EPI != kEpiRawI32)
        if (p.persist > 0) return launch_lds_cfg<I8, EPI, 8, 4, 2, 3, 0, 128, 2, 4, true>(p, max_tiles, stream);
      // W13 (gate/up pairs) on 4-wave workgroups, two per CU (2 x 2 waves of
      // 128 x 96, 72 KB of LDS): another workgroup's K loop overlaps each
      // item's epilogue (C3 W13 0.938 -> 0.927 ms, C4 0.455 -> 0.417 ms). W2
      // ran slower that way (C3 0.530 -> 0.586 ms) and keeps 8 waves.
      if constexpr (epi_pair(EPI))
        return launch_lds_cfg<I8, EPI, 8, 6, 2, 3, 0, 64, 2, 2>(p, max_tiles, stream);
      // i8gemm (one expert, the row tiles known on the host): 256 x 256
      // workgroups where they need fewer rounds of the CUs than 256 x 384
      // ones, weighing a round by its channels and the 128 x 64 wave tile's
      // ~6% lower MFMA rate (the LDS loop probe: 3.87 vs 4.12 POPS). DeepSeek
      // V4's wo_b ([7168, 16384]) on 256 CUs: 448 items in 2 rounds instead
      // of 304 in 2, at 1024 / 2048 / 4096 rows 0.295 / 0.337 / 0.636 ->
      // 0.224 / 0.290 / 0.562 ms. The pair's [24576, 1536] takes 256 x 384
      // (1024 items in 4 rounds, not 1536 in 6) and its [8192, 1536] 256 x
      // 256: 0.317 -> 0.294 ms at 4096 rows, against 0.310 / 0.294 with
      // either width for both. max_tiles must be the exact row-tile count.
      // 4-wave workgroups two per CU were no faster.
      if constexpr (EPI == kEpiI8Gemm) {
        if (p.cus > 0 && p.n_groups == 1) {
          const int64_t sp = p.k_total > 0 ? ceil_div(p.k_total, p.k_chunks) : 1;  // K splits
          const int64_t r384 = ceil_div(max_tiles * ceil_div(p.n_tiles, 24) * sp, p.cus);
          const int64_t r256 = ceil_div(max_tiles * ceil_div(p.n_tiles, 16) * sp, p.cus);
          if (r256 * 16 * 106 < r384 * 24 * 100)
            return launch_lds_cfg<I8, EPI, 8, 4, 2, 3, 0, 128, 2, 4>(p, max_tiles, stream);
        }
      }
      return launch_lds_cfg<I8, EPI, 8, 6, 2, 3, 0, 128>(p, max_tiles, stream);
    default:
      return fail(FCMOE_EINVAL, "unsupported LDS tile rows");
  }
}

// W8A16 prefill tiles. The int8 -> bf16 widening is VALU work on the MFMAs'
// SIMD, done once per chunk and weight tile, so each wave covers many row
// fragments against few tiles (two bf16 MFMAs per pair per chunk): the 128-row
// tile runs 1 x 8 waves of 8 x 4, the 256-row tile 2 x 4 waves of 8 x 4, the
// 192-row tile 1 x 8 waves of 12 row fragments x 2 tiles, which widens every
// weight tile once per workgroup (2 x 4 waves of 6 x 4 widened each tile in
// both wave rows: DSv3 shape at T=4096, W13 1.24 -> 1.17 ms, W2 0.68 -> 0.66). As in the int8 classes, the 128/192-row weights stream
// nontemporal (one row tile per expert) and the 256-row ones stay cached
// (their experts' row tiles re-read them).
template <int EPI>
int launch_lds_w8(int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  constexpr int kNT = 2;
  switch (bm) {
    case 128:
      return launch_lds_cfg<false, EPI, 8, 4, 2, 3, kNT, 128, 1, 8>(p, max_tiles, stream);
    case 192:
      return launch_lds_cfg<false, EPI, 12, 2, 2, 3, kNT, 128, 1, 8>(p, max_tiles, stream);
    case 256:
      return launch_lds_cfg<false, EPI, 8, 4, 2, 3, 0, 128, 2, 4>(p, max_tiles, stream);
    default:
      return fail(FCMOE_EINVAL, "W8A16 LDS tiles are 128, 192 or 256 rows");
  }
}

}  // namespace

#if FCMOE_DIAG & 4
// Diagnostic builds: the item trace (2 x 256 workgroups x 64 items x 4
// 64-bit words) copied to host (write = 0), or overwritten from host (write =
// 1: the caller passes zeros to clear it).
extern "C" int fcmoe_diag_item_trace(void* host, int write) {
  const hipError_t e = write ? hipMemcpyToSymbol(HIP_SYMBOL(g_item_trace), host, sizeof(g_item_trace))
                             : hipMemcpyFromSymbol(host, HIP_SYMBOL(g_item_trace), sizeof(g_item_trace));
  return e == hipSuccess ? 0 : -1;
}
#endif

int gemm_lds_launch(int epi, int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  switch (epi) {
    case kEpiRawI32:
      return launch_lds_bm<true, kEpiRawI32>(bm, p, max_tiles, stream);
    case kEpiW13SwigluI8:
      return launch_lds_bm<true, kEpiW13SwigluI8>(bm, p, max_tiles, stream);
    case kEpiW2RouteI8:
      return launch_lds_bm<true, kEpiW2RouteI8>(bm, p, max_tiles, stream);
    case kEpiI8Gemm:
      return launch_lds_bm<true, kEpiI8Gemm>(bm, p, max_tiles, stream);
    case kEpiW13ActBf16:
      return launch_lds_bm<false, kEpiW13ActBf16>(bm, p, max_tiles, stream);
    case kEpiRawF32Bias:
      return launch_lds_bm<false, kEpiRawF32Bias>(bm, p, max_tiles, stream);
    case kEpiW2RouteBf16:
      return launch_lds_bm<false, kEpiW2RouteBf16>(bm, p, max_tiles, stream);
    case kEpiW13ActW8:
      return launch_lds_w8<kEpiW13ActW8>(bm, p, max_tiles, stream);
    case kEpiW2RouteW8:
      return launch_lds_w8<kEpiW2RouteW8>(bm, p, max_tiles, stream);
    default:
      return fail(FCMOE_EINVAL, "unknown epilogue");
  }
}

}  // namespace fcmoe
