// fcmoe_gemm_lds_common.h -- pieces shared by the LDS-staged grouped GEMMs
// (fcmoe_gemm_lds.hip: 2 waves per SIMD, accumulators in VGPRs;
// fcmoe_gemm_pipe.hip: 1 wave per SIMD, accumulators in AGPRs): buffer
// resources, counted waits, the XCD-aware work order of persistent and
// non-persistent launches, and the staged W8A8 epilogues.
#pragma once

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

// Accumulators held in AGPRs (FENCE): each 16-row fragment's accumulators
// are moved to VGPRs through the wave's LDS area `acc_stage` (16 bytes per
// lane and tile, written straight from the AGPRs by an asm ds_write and read
// back), one fragment at a time. The compiler sees no VGPR use of an
// accumulator after the K loop, so it leaves them in AGPRs instead of copying
// every one to VGPRs where the loop ends (more than a wave's VGPRs).
template <int FN>
__device__ __forceinline__ void acc_row_to_vgprs(const v4i (&acc)[FN], lds_u8_ptr acc_stage, int lane,
                                                 v4i (&out)[FN]) {
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const uint32_t addr = (uint32_t)(uintptr_t)(acc_stage + (j * kWave + lane) * 16);
    asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "a"(acc[j]) : "memory");
  }
#pragma unroll
  for (int j = 0; j < FN; ++j)
    out[j] = *(__attribute__((address_space(3))) const v4i*)(acc_stage + (j * kWave + lane) * 16);
}

template <int EPI, int FM, int FN, bool FENCE = false>
__device__ __forceinline__ void staged_epilogue(const GemmParams& p, const v4i (&acc)[FM][FN],
                                                const int64_t (&gtile)[FN], const bool (&tvalid)[FN], int row_base,
                                                int rows, int pos0, int expert, int lane, const EpiMeta& m,
                                                lds_u8_ptr slice, lds_u8_ptr acc_stage = nullptr) {
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
      v4i av[FN];
      if constexpr (FENCE) acc_row_to_vgprs<FN>(acc[i], acc_stage, lane, av);
      const v4i(&ar)[FN] = FENCE ? av : acc[i];
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
            gate[b][j] = fminf((float)ar[j][q0 + b] * (xs * cg[j]), 10.0f);
            up[b][j] = fmaxf(fminf((float)ar[j + HP][q0 + b] * (xs * cu[j]), 10.0f), -10.0f);
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
      v4i av[FN];
      if constexpr (FENCE) acc_row_to_vgprs<FN>(acc[i], acc_stage, lane, av);
      const v4i(&ar)[FN] = FENCE ? av : acc[i];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = rbase + rq + q;
        const float rs = m.rs[r < rows ? r : rows - 1];
#pragma unroll
        for (int j = 0; j < FN; ++j)
          *(__attribute__((address_space(3))) float*)(slice + (rq + q) * RS + (j * 16 + col) * 4) =
              (float)ar[j][q] * (rs * cs[j]);
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

// Channel blocks per row tile of a workgroup whose waves hold FN 16-channel
// tiles (W13: FN/2 gate/up pairs).
template <int EPI>
int64_t lds_blocks(int wn, int fn, const GemmParams& p) {
  constexpr bool PAIR = epi_pair(EPI);
  const int64_t per_block = PAIR ? (int64_t)wn * (fn / 2) : (int64_t)wn * fn;
  const int64_t units = PAIR ? p.n_tiles : (int64_t)p.n_groups * p.n_tiles;
  return ceil_div(units, per_block);
}

}  // namespace

}  // namespace fcmoe
