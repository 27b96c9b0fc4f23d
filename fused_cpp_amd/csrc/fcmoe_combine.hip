// fcmoe_combine.hip -- routing-weighted un-permute combine.
//
// out[t, h] = bf16(sum over slots of route_out[t*kt + s, h] * w[t*kt + s]).
// Ordered mode is the W8A8 merge: acc = fma(route, w, acc) for s = 0..kt-1
// (csrc/moe/arm/i8mm_w8a8/kernels.cpp:674-688) and the BF16 merge for top-k
// outside {2,4,6,8}. Tree mode is the BF16 SVE merge for top-k in {2,4,6,8}:
// products route*w, then adjacent-pair additions splitting each range at its
// largest power of two below its length, ((0+1)+(2+3))+(4+5) for 6
// (csrc/moe/arm/sve_bf16/route_merge.cpp:47-86). skip_weighted copies the
// single route (naive.py:392-393). One thread per output element: consecutive
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

template <int K>
__device__ __forceinline__ float tree_merge(const float* route_out, const float* w, int64_t r0, int64_t hidden,
                                            int64_t h) {
  float v[K];
#pragma unroll
  for (int s = 0; s < K; ++s) v[s] = route_out[(r0 + s) * hidden + h] * w[r0 + s];
  return TreeSum<0, K>::run(v);
}

// VW output channels per thread (VW = 4 when hidden % 4 == 0: 16-byte route
// loads, 8-byte bf16 stores; else 1). Each channel's arithmetic is identical
// to the scalar form.
template <int VW>
__global__ __launch_bounds__(256) void combine_kernel(const float* route_out, const float* route_weight,
                                                       const int32_t* route_pos, int64_t tokens, int kt,
                                                       int64_t hidden, int tree, int skip_weighted, uint16_t* out) {
  const int64_t t = blockIdx.y;
  const int64_t h0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VW;
  if (t >= tokens || h0 >= hidden) return;
  const int64_t r0 = t * kt;
  float acc[VW];
#pragma unroll
  for (int v = 0; v < VW; ++v) acc[v] = 0.0f;
  auto load = [&](int64_t r, float (&dst)[VW]) {
    if constexpr (VW == 4) {
      const float4 q = *(const float4*)(route_out + r * hidden + h0);
      dst[0] = q.x;
      dst[1] = q.y;
      dst[2] = q.z;
      dst[3] = q.w;
    } else {
      dst[0] = route_out[r * hidden + h0];
    }
  };
  if (skip_weighted) {
    if (route_pos[r0] >= 0) load(r0, acc);
  } else if (tree) {
#pragma unroll
    for (int v = 0; v < VW; ++v) {
      switch (kt) {
        case 2:
          acc[v] = tree_merge<2>(route_out, route_weight, r0, hidden, h0 + v);
          break;
        case 4:
          acc[v] = tree_merge<4>(route_out, route_weight, r0, hidden, h0 + v);
          break;
        case 6:
          acc[v] = tree_merge<6>(route_out, route_weight, r0, hidden, h0 + v);
          break;
        default:
          acc[v] = tree_merge<8>(route_out, route_weight, r0, hidden, h0 + v);
          break;
      }
    }
  } else {
    for (int s = 0; s < kt; ++s) {
      const int64_t r = r0 + s;
      if (route_pos[r] < 0) continue;
      const float w = route_weight[r];
      float v4[VW];
      load(r, v4);
#pragma unroll
      for (int v = 0; v < VW; ++v) acc[v] = __builtin_fmaf(v4[v], w, acc[v]);
    }
  }
  if constexpr (VW == 4) {
    const uint32_t lo = (uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
    *(uint2*)(out + t * hidden + h0) = make_uint2(lo, hi);
  } else {
    out[t * hidden + h0] = f32_to_bf16(acc[0]);
  }
}

}  // namespace

int combine_launch(const float* route_out, const float* route_weight, const int32_t* route_pos, int64_t tokens,
                   int64_t kt, int64_t hidden, int tree, int skip_weighted, uint16_t* out, hipStream_t stream) {
  if (tokens <= 0) return FCMOE_OK;
  if (tokens > 65535) return fail(FCMOE_EINVAL, "too many tokens");
  if (hidden % 4 == 0)
    hipLaunchKernelGGL(combine_kernel<4>, dim3((unsigned)ceil_div(hidden / 4, 256), (unsigned)tokens), dim3(256), 0,
                       stream, route_out, route_weight, route_pos, tokens, (int)kt, hidden, tree, skip_weighted, out);
  else
    hipLaunchKernelGGL(combine_kernel<1>, dim3((unsigned)ceil_div(hidden, 256), (unsigned)tokens), dim3(256), 0,
                       stream, route_out, route_weight, route_pos, tokens, (int)kt, hidden, tree, skip_weighted, out);
  return check_launch("combine");
}

}  // namespace fcmoe
