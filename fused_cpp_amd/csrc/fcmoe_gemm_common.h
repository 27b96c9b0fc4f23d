// fcmoe_gemm_common.h -- pieces shared by the grouped-GEMM kernels
// (fcmoe_gemm.hip: register-ring kernels; fcmoe_gemm_lds.hip: LDS-staged
// prefill kernel): MFMA wrappers, bf16-path activations, the LDS barrier and
// the fused epilogues.
//
// Accumulator layout (both kernels): acc[i][j] is the 16x16 block of row
// fragment i and channel tile j; lane l, register q holds row
// row_base + 16 i + 4 (l / 16) + q and column l % 16 of tile gtile[j].
#pragma once

#include "fcmoe_device.h"
#include "fcmoe_internal.h"

namespace fcmoe {
namespace {

template <bool I8>
struct Acc;
template <>
struct Acc<true> {
  typedef v4i type;
};
template <>
struct Acc<false> {
  typedef v4f type;
};

__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma(v8bf a, v8bf b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float act_bf16_mode(float g, float u, int mode) {
  if (mode == FCMOE_ACT_SILU_CLAMP10) {
    g = fminf(g, 10.0f);
    u = fmaxf(fminf(u, 10.0f), -10.0f);
  }
  if (mode == FCMOE_ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752440f)) * u;
  return silu_f(g) * u;
}

// Barrier for the LDS A buffers: waits only for this wave's LDS traffic
// (lgkmcnt), not for the weight loads still in flight (a __syncthreads fence
// would also drain vmcnt and empty the prefetch ring).
// The builtin (not inline asm) lets the compiler's wait-count pass see the
// wait, so it does not wait again for LDS reads this one already covered.
// gfx9 s_waitcnt immediate: vmcnt [3:0]+[15:14], expcnt [6:4], lgkmcnt
// [11:8]; 0xC07F = lgkmcnt(0), the other counters unconstrained.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
}

// W13 epilogues pair gate and up tiles; W8A16 epilogues stream int8 weights
// against bf16 activations.
__host__ __device__ constexpr bool epi_pair(int epi) {
  return epi == kEpiW13SwigluI8 || epi == kEpiW13ActBf16 || epi == kEpiW13ActW8;
}
__host__ __device__ constexpr bool epi_w8(int epi) { return epi == kEpiW13ActW8 || epi == kEpiW2RouteW8; }

// 16 int8 weights -> two bf16 MFMA operands (bytes 0-7, bytes 8-15), as
// packed bf16 pairs in 32-bit words. Exact: each byte converts to fp32 with
// one sign-extending byte-select v_cvt_f32_i32 (SDWA), and |q| <= 128 has at
// most 8 significant bits, so the high 16 bits of the fp32 value are its bf16
// value (v_perm packs two). Six VALU ops per 4 bytes (a bias-to-unsigned form
// took twelve).
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
__device__ __forceinline__ void i8x16_to_bf16(v4i b, v4i& lo, v4i& hi) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t u = (uint32_t)b[w];
    const float f0 = (float)(int8_t)u;
    const float f1 = (float)(int8_t)(u >> 8);
    const float f2 = (float)(int8_t)(u >> 16);
    const float f3 = (float)((int32_t)u >> 24);
    const int p0 = (int)bf16_pair(f0, f1), p1 = (int)bf16_pair(f2, f3);
    if (w < 2) {
      lo[2 * w] = p0;
      lo[2 * w + 1] = p1;
    } else {
      hi[2 * (w - 2)] = p0;
      hi[2 * (w - 2) + 1] = p1;
    }
  }
}

// Fused epilogues. W13 pairs: tiles j < FN/2 are gate tiles and tile
// j + FN/2 is the matching up tile (same channels of the other group).
//
// Per-column values (channels, scales, biases) are loaded once and per-row
// values (positions, routes, row scales) once per 16-row fragment, ahead of
// that fragment's stores: the output may alias those arrays as far as the
// compiler knows, so a load left between stores would wait for each store.
// Channels, positions and routes fit in 32 bits (checked by the launchers).
//
// Staged metadata (LM): the LDS kernel loads the tile's per-row values (row
// scale, output row) and per-channel scales into LDS before its K loop
// (EpiMeta). Loaded here instead, a row value load issued after a
// fragment's stores waits for those stores too (vmcnt counts both, in
// order), and the W13 row scale is a dependent pair of loads: six fragments
// made the epilogue a chain of ~30 memory round trips.
// The pointers are typed as LDS (address space 3): as generic pointers the
// reads compile to flat loads, which count in vmcnt as well and may alias
// the output, so each one waited for every store before it.
typedef __attribute__((address_space(3))) const float* lds_cfloat_ptr;
typedef __attribute__((address_space(3))) const int* lds_cint_ptr;
struct EpiMeta {
  lds_cfloat_ptr rs;  // [BM] row scale (W13: x scale of the row's token)
  lds_cint_ptr orow;  // [BM] output row (W2: flat route; else sorted position)
  lds_cfloat_ptr cs;  // [NT * 16] per-channel scale of channel tile slot s
  int cbase;          // this wave's first slot
};

// Epilogues whose per-channel values are scales (staged by the LDS kernel);
// the bias epilogues load their biases here (one round trip, before any
// store).
__host__ __device__ constexpr bool epi_col_scale(int epi) {
  return epi == kEpiW13SwigluI8 || epi == kEpiW2RouteI8 || epi == kEpiI8Gemm;
}
__host__ __device__ constexpr bool epi_route(int epi) {
  return epi == kEpiW2RouteI8 || epi == kEpiW2RouteBf16 || epi == kEpiW2RouteW8;
}

template <bool I8, int EPI, int FM, int FN, bool LM = false>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, const typename Acc<I8>::type (&acc)[FM][FN],
                                              const int64_t (&gtile)[FN], const bool (&tvalid)[FN], int row_base,
                                              int rows, int pos0, int expert, int lane, const EpiMeta& m = {}) {
  const int col = lane % 16;
  // tile-local row of (fragment i, register q), clamped like row_of
  auto lrow = [&](int i, int q) -> int {
    const int r = row_base + i * 16 + (lane / 16) * 4 + q;
    return r < rows ? r : rows - 1;
  };
  auto row_of = [&](int i, int q, bool* ok) -> int {
    const int r = row_base + i * 16 + (lane / 16) * 4 + q;
    *ok = r < rows;
    return pos0 + (r < rows ? r : rows - 1);  // clamped: loads stay in range
  };
  if constexpr (epi_pair(EPI)) {
    constexpr int HP = FN / 2;
    const int64_t n = p.n;  // 2F logical
    const uint32_t ftab = EPI == kEpiW13SwigluI8 ? fexpa_table_lane() : 0u;
    int f[HP];
    bool fv[HP];
    float cg[HP], cu[HP];  // W13 int8 / W8A16: gate / up channel scales; bf16: biases
#pragma unroll
    for (int j = 0; j < HP; ++j) {
      f[j] = (int)(gtile[j] * 16 + col);  // gate channel (group 0)
      fv[j] = tvalid[j] && f[j] < p.n_half;
      const int64_t fc = fv[j] ? f[j] : 0;
      if constexpr (LM && epi_col_scale(EPI)) {
        cg[j] = m.cs[(m.cbase + j) * 16 + col];
        cu[j] = m.cs[(m.cbase + j + HP) * 16 + col];
      } else if constexpr (EPI == kEpiW13SwigluI8 || EPI == kEpiW13ActW8) {
        cg[j] = p.scale_col[(int64_t)expert * n + fc];
        cu[j] = p.scale_col[(int64_t)expert * n + p.n_half + fc];
      } else {
        cg[j] = p.bias ? p.bias[(int64_t)expert * n + fc] : 0.0f;
        cu[j] = p.bias ? p.bias[(int64_t)expert * n + p.n_half + fc] : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int pos[4];
      bool rok[4];
      float xs[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pos[q] = row_of(i, q, &rok[q]);
        if constexpr (EPI == kEpiW13SwigluI8) {
          if constexpr (LM)
            xs[q] = m.rs[lrow(i, q)];
          else
            xs[q] = p.scale_row[p.row_map ? p.row_map[pos[q]] : pos[q]];
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < HP; ++j) {
          float ya = 0.0f;  // |y| of this lane's channel (0 past F or past the tile's rows)
          if constexpr (EPI == kEpiW13SwigluI8) {
            // w13_epilogue, csrc/moe/arm/i8mm_w8a8/kernels.cpp:230-246. Evaluated
            // on every lane (operands are clamped in range) so the table lookup's
            // cross-lane read sees all lanes active; only the store is guarded.
            float gate = (float)acc[i][j][q] * (xs[q] * cg[j]);
            float up = (float)acc[i][j + HP][q] * (xs[q] * cu[j]);
            gate = fminf(gate, 10.0f);
            up = fmaxf(fminf(up, 10.0f), -10.0f);
            const float ex = fexpa_exp_neg_v(gate, ftab);
            const float y = (gate * up) / (ex + 1.0f);
            if (rok[q] && fv[j]) {
              const uint16_t yb = f32_to_bf16(y);
              ((uint16_t*)p.out)[(int64_t)pos[q] * p.ldo + f[j]] = yb;
              ya = fabsf(bf16_to_f32(yb));
            }
          } else if (rok[q] && fv[j]) {
            float y;
            if constexpr (EPI == kEpiW13ActW8) {
              // x . (q * s) accumulated as (x . q) * s in fp32
              y = act_bf16_mode(acc[i][j][q] * cg[j], acc[i][j + HP][q] * cu[j], p.activation);
            } else {
              float gate = acc[i][j][q];
              float up = acc[i][j + HP][q];
              if (p.bias) {
                gate = gate + cg[j];
                up = up + cu[j];
              }
              y = act_bf16_mode(gate, up, p.activation);
            }
            const uint16_t yb = f32_to_bf16(y);
            ((uint16_t*)p.out)[(int64_t)pos[q] * p.ldo + f[j]] = yb;
          }
          if constexpr (EPI == kEpiW13SwigluI8) {
            // Maximum of |y| over this 16-channel gate tile (lanes reconverged
            // for the shuffle); one plain store per (row, tile): every gate tile
            // of a row is written by exactly one wave, so no atomics.
            const float amax = max16(ya);
            if (rok[q] && tvalid[j] && col == 0) p.rowpart[(int64_t)pos[q] * p.n_tiles + gtile[j]] = amax;
          }
        }
      }
    }
  } else {
    constexpr bool ROUTE = EPI == kEpiW2RouteI8 || EPI == kEpiW2RouteBf16 || EPI == kEpiW2RouteW8;
    constexpr bool ROWSCALE = EPI == kEpiW2RouteI8 || EPI == kEpiI8Gemm;
    int ch[FN], dch[FN];
    bool cv[FN];
    float cs[FN], cb[FN];  // column scale, column bias
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t g = gtile[j] / p.n_tiles;
      const int64_t t = gtile[j] - g * p.n_tiles;
      const int64_t cin = t * 16 + col;
      cv[j] = tvalid[j] && cin < p.n_half;
      ch[j] = cv[j] ? (int)(g * p.n_half + cin) : 0;          // logical channel
      dch[j] = EPI == kEpiRawF32Bias ? (int)(gtile[j] * 16 + col) : ch[j];  // RawF32Bias: packed order
      cs[j] = 0.0f;
      cb[j] = 0.0f;
      if constexpr (LM && epi_col_scale(EPI)) {
        cs[j] = m.cs[(m.cbase + j) * 16 + col];
      } else if constexpr (EPI == kEpiW2RouteI8 || EPI == kEpiW2RouteW8) {
        cs[j] = p.scale_col[(int64_t)expert * p.n + ch[j]];
      } else if constexpr (EPI == kEpiI8Gemm) {
        cs[j] = p.scale_col[ch[j]];
      }
      if constexpr (EPI == kEpiI8Gemm) {
        if (p.bias) cb[j] = p.bias[ch[j]];
      }
      if constexpr (EPI == kEpiRawF32Bias || EPI == kEpiW2RouteBf16) {
        if (p.bias) cb[j] = p.bias[(int64_t)expert * p.n + ch[j]];
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int orow[4];  // output row: sorted position or flat route
      bool rok[4];
      float rs[4];  // row scale
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pos = row_of(i, q, &rok[q]);
        if constexpr (LM) {
          orow[q] = m.orow[lrow(i, q)];
          rs[q] = ROWSCALE ? m.rs[lrow(i, q)] : 0.0f;
        } else {
          orow[q] = ROUTE ? p.sorted_routes[pos] : pos;
          rs[q] = ROWSCALE ? p.scale_row[pos] : 0.0f;
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (!rok[q]) continue;
        const int64_t obase = (int64_t)orow[q] * p.ldo;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          if (!cv[j]) continue;
          if constexpr (EPI == kEpiRawI32) {
            ((int32_t*)p.out)[obase + ch[j]] = (int32_t)acc[i][j][q];
          } else if constexpr (EPI == kEpiW2RouteI8) {
            // store_w2, csrc/moe/arm/i8mm_w8a8/kernels.cpp:248-257.
            ((float*)p.out)[obase + ch[j]] = (float)acc[i][j][q] * (rs[q] * cs[j]);
          } else if constexpr (EPI == kEpiI8Gemm) {
            // write_scaled_output, csrc/i8gemm.cpp:148-164 (left to right).
            float v = (float)acc[i][j][q] * rs[q] * cs[j];
            if (p.bias) v = v + cb[j];
            if (p.out_bf16)
              ((uint16_t*)p.out)[obase + ch[j]] = f32_to_bf16(v);
            else
              ((float*)p.out)[obase + ch[j]] = v;
          } else if constexpr (EPI == kEpiW2RouteW8) {
            ((float*)p.out)[obase + ch[j]] = acc[i][j][q] * cs[j];
          } else {  // kEpiRawF32Bias, kEpiW2RouteBf16
            float v = acc[i][j][q];
            if (p.bias) v = v + cb[j];
            ((float*)p.out)[obase + dch[j]] = v;
          }
        }
      }
    }
  }
}

}  // namespace
}  // namespace fcmoe
