// fcmoe_combine.hip -- routing-weighted un-permute combine.
//
// out[t, h] = bf16(sum over slots of route_out[t*kt + s, h] * w[t*kt + s]).
// Ordered mode is the W8A8 merge: acc = fma(route, w, acc) for s = 0..kt-1
// (csrc/moe/arm/i8mm_w8a8/kernels.cpp:674-688) and the BF16 merge for top-k
// outside {2,4,6,8}. Tree mode is the BF16 SVE merge for top-k in {2,4,6,8}:
// products route*w, then adjacent-pair additions splitting each range at its
// largest power of two below its length, ((0+1)+(2+3))+(4+5) for 6
// (csrc/moe/arm/sve_bf16/route_merge.cpp:47-86). skip_weighted copies the
// single route (naive.py:259-261). One thread per output element: consecutive
// threads read consecutive h of each route row (HBM-bound, coalesced).
#include "fcmoe_device.h"
#include "fcmoe_internal.h"

namespace fcmoe {

namespace {

template <int Begin, int Count>
struct TreeSum {
  __device__ __forceinline__ static float run(const float* v) {
    constexpr int P = Count > 1 ? [] {
      int p = 1;
      while ((p << 1) < Count) p <<= 1;
      return p;
    }()
                                : 1;
    return TreeSum<Begin, P>::run(v) + TreeSum<Begin + P, Count - P>::run(v);
  }
};
template <int Begin>
struct TreeSum<Begin, 1> {
  __device__ __forceinline__ static float run(const float* v) { return v[Begin]; }
};

// A dropped (invalid) route's row was never written: its leaf is 0 by a
// select, so whatever the row holds (NaN included) cannot reach the sum.
template <int K>
__device__ __forceinline__ float tree_merge(const float* route_out, const float* w, const int32_t* route_pos,
                                            int64_t r0, int64_t hidden, int64_t h) {
  float v[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    const float prod = route_out[(r0 + s) * hidden + h] * w[r0 + s];
    v[s] = route_pos[r0 + s] >= 0 ? prod : 0.0f;
  }
  return TreeSum<0, K>::run(v);
}

// VW output channels per thread (VW = 4 when hidden % 4 == 0: 16-byte route
// loads, 8-byte bf16 stores; else 1). Each channel's arithmetic is identical
// to the scalar form.
// Route rows are read exactly once: nontemporal loads stream them past the
// caches. The ordered merge issues every load of up to kSlotBatch slots (row,
// position, weight) before its FMA chain (slot order unchanged), so a thread
// waits one memory round trip per batch. A row is loaded whatever its
// position says (rows t*kt + s always lie inside route_out) and a dropped
// route's row, which was never written, is left out by the select, not by
// a multiply. Tokens run grid-stride over y.
constexpr int kSlotBatch = 16;
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

template <int VW>
__global__ __launch_bounds__(256) void combine_kernel(const float* route_out, const float* route_weight,
                                                       const int32_t* route_pos, int64_t tokens, int kt,
                                                       int64_t hidden, int tree, int skip_weighted, uint16_t* out) {
  const int64_t h0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VW;
  if (h0 >= hidden) return;
  for (int64_t t = blockIdx.y; t < tokens; t += gridDim.y) {
  const int64_t r0 = t * kt;
  float acc[VW];
#pragma unroll
  for (int v = 0; v < VW; ++v) acc[v] = 0.0f;
  auto load = [&](int64_t r, float (&dst)[VW]) {
    if constexpr (VW == 4) {
      const v4f q = __builtin_nontemporal_load((const v4f*)(route_out + r * hidden + h0));
      dst[0] = q.x;
      dst[1] = q.y;
      dst[2] = q.z;
      dst[3] = q.w;
    } else {
      dst[0] = __builtin_nontemporal_load(route_out + r * hidden + h0);
    }
  };
  if (skip_weighted) {
    if (route_pos[r0] >= 0) load(r0, acc);
  } else if (tree) {
#pragma unroll
    for (int v = 0; v < VW; ++v) {
      switch (kt) {
        case 2:
          acc[v] = tree_merge<2>(route_out, route_weight, route_pos, r0, hidden, h0 + v);
          break;
        case 4:
          acc[v] = tree_merge<4>(route_out, route_weight, route_pos, r0, hidden, h0 + v);
          break;
        case 6:
          acc[v] = tree_merge<6>(route_out, route_weight, route_pos, r0, hidden, h0 + v);
          break;
        default:
          acc[v] = tree_merge<8>(route_out, route_weight, route_pos, r0, hidden, h0 + v);
          break;
      }
    }
  } else {
    for (int s0 = 0; s0 < kt; s0 += kSlotBatch) {
      float v[kSlotBatch][VW];
      float w[kSlotBatch];
      int pos[kSlotBatch];
#pragma unroll
      for (int u = 0; u < kSlotBatch; ++u) {
        const int64_t r = r0 + s0 + u;
        pos[u] = -1;
        w[u] = 0.0f;
        if (s0 + u < kt) {  // uniform over the grid
          pos[u] = route_pos[r];
          w[u] = route_weight[r];
          load(r, v[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < kSlotBatch; ++u)
        if (pos[u] >= 0) {  // dropped (invalid) routes hold no row
#pragma unroll
          for (int c = 0; c < VW; ++c) acc[c] = __builtin_fmaf(v[u][c], w[u], acc[c]);
        }
    }
  }
  if constexpr (VW == 4) {
    const uint32_t lo = (uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
    // nontemporal: the caller reads the output later, after other work
    // (C4 combine 0.368 -> 0.348 ms)
    __builtin_nontemporal_store((v2u){lo, hi}, (v2u*)(out + t * hidden + h0));
  } else {
    out[t * hidden + h0] = f32_to_bf16(acc[0]);
  }
  }
}

}  // namespace

int combine_launch(const float* route_out, const float* route_weight, const int32_t* route_pos, int64_t tokens,
                   int64_t kt, int64_t hidden, int tree, int skip_weighted, uint16_t* out, hipStream_t stream) {
  if (tokens <= 0) return FCMOE_OK;
  const unsigned ty = (unsigned)(tokens < 65535 ? tokens : 65535);  // grid.y limit; the kernel strides over y
  if (hidden % 4 == 0)
    hipLaunchKernelGGL(combine_kernel<4>, dim3((unsigned)ceil_div(hidden / 4, 256), ty), dim3(256), 0,
                       stream, route_out, route_weight, route_pos, tokens, (int)kt, hidden, tree, skip_weighted, out);
  else
    hipLaunchKernelGGL(combine_kernel<1>, dim3((unsigned)ceil_div(hidden, 256), ty), dim3(256), 0,
                       stream, route_out, route_weight, route_pos, tokens, (int)kt, hidden, tree, skip_weighted, out);
  return check_launch("combine");
}

}  // namespace fcmoe
