// fcmoe_router.hip -- top-k softmax router: logits [T, E] fp32 -> topk_ids
// [T, k] and topk_weights [T, k] fp32.
//
// The reference receives ids and weights from its caller
// (src/fused_cpp/moe/bf16_tiled.py:676-681; the vLLM adapter routes with
// softmax -> top-k -> renormalise -> routed scaling,
// docs/vllm_bf16_tiled_moe_integration.md:75-87). This kernel is that caller
// step on the GPU so a MoE layer runs without a host round trip.
//
// One wavefront per token. Lane l holds experts l, l+64, ... (coalesced
// loads); the softmax max and sum are butterfly reductions; the k winners are
// found by k rounds of a wave argmax over (logit, lower id on ties), since
// softmax is monotonic in the logit. Weights: p = exp(x - max) / sum, then
// optionally p / sum(selected p), then * scale. Ids come out in descending
// logit order.
#include "fcmoe_device.h"
#include "fcmoe_internal.h"

namespace fcmoe {

namespace {

constexpr int kRouterWaves = 4;  // tokens per workgroup

template <int VPL>  // logits per lane: experts <= 64 * VPL
__global__ __launch_bounds__(kRouterWaves * kWave) void router_topk_kernel(const float* __restrict__ logits,
                                                                           int64_t tokens, int experts, int top_k,
                                                                           int renorm, float scale, void* ids,
                                                                           int ids_is_i64, float* weights) {
  const int lane = threadIdx.x % kWave;
  const int64_t t = (int64_t)blockIdx.x * kRouterWaves + threadIdx.x / kWave;
  if (t >= tokens) return;  // whole wave exits together
  const float* row = logits + t * experts;

  float v[VPL];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + i * kWave;
    v[i] = e < experts ? row[e] : -INFINITY;
    m = fmaxf(m, v[i]);
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + i * kWave;
    if (e < experts) s += expf(v[i] - m);
  }
  s = wave_sum(s);

  // k rounds of argmax over the experts not chosen yet (a per-lane bit per
  // value slot). NaN logits never win: every comparison with NaN is false.
  // When no candidate is left (the rest are NaN), the lowest unchosen id is
  // taken, so the k ids of a row are always distinct.
  float psel = 0.0f;  // lane s of the wave keeps winner s's probability
  int esel = 0;
  float psum = 0.0f;
  uint32_t chosen = 0;
  for (int r = 0; r < top_k; ++r) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
    int first_free = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = lane + i * kWave;
      if (e < experts && !((chosen >> i) & 1u)) {
        if (e < first_free) first_free = e;
        if (v[i] > bv || (v[i] == bv && e < be)) {
          bv = v[i];
          be = e;
        }
      }
    }
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oe = __shfl_xor(be, off);
      if (ov > bv || (ov == bv && oe < be)) {
        bv = ov;
        be = oe;
      }
      first_free = min(first_free, __shfl_xor(first_free, off));
    }
    if (be == 0x7fffffff) {  // only NaN logits left
      be = first_free;
      bv = -INFINITY;
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (lane + i * kWave == be) chosen |= 1u << i;
    const float p = expf(bv - m) / s;
    psum += p;
    if (lane == r) {
      psel = p;
      esel = be;
    }
  }
  if (lane < top_k) {
    float w = renorm ? psel / psum : psel;
    w = w * scale;
    weights[t * top_k + lane] = w;
    if (ids_is_i64)
      ((int64_t*)ids)[t * top_k + lane] = esel;
    else
      ((int32_t*)ids)[t * top_k + lane] = esel;
  }
}

}  // namespace

}  // namespace fcmoe

using namespace fcmoe;

extern "C" int fcmoe_router_topk(const float* logits, int64_t tokens, int64_t experts, int64_t top_k,
                                 int renormalize, float scale, void* topk_ids, int ids_is_i64,
                                 float* topk_weights, hipStream_t stream) {
  if (tokens < 0 || experts <= 0 || experts > 1024 || top_k <= 0 || top_k > experts || top_k > kWave)
    return fail(FCMOE_EINVAL, "router_topk: need 0 < top_k <= min(experts, 64), experts <= 1024");
  if (tokens == 0) return FCMOE_OK;
  if (!logits || !topk_ids || !topk_weights) return fail(FCMOE_EINVAL, "router_topk: NULL pointer");
  const int64_t grid = ceil_div(tokens, (int64_t)kRouterWaves);
  if (grid > INT32_MAX) return fail(FCMOE_EINVAL, "router_topk: too many tokens");
  const dim3 g((unsigned)grid), b(kRouterWaves * kWave);
  const int E = (int)experts, K = (int)top_k;
  if (experts <= 64)
    hipLaunchKernelGGL(router_topk_kernel<1>, g, b, 0, stream, logits, tokens, E, K, renormalize, scale, topk_ids,
                       ids_is_i64, topk_weights);
  else if (experts <= 128)
    hipLaunchKernelGGL(router_topk_kernel<2>, g, b, 0, stream, logits, tokens, E, K, renormalize, scale, topk_ids,
                       ids_is_i64, topk_weights);
  else if (experts <= 256)
    hipLaunchKernelGGL(router_topk_kernel<4>, g, b, 0, stream, logits, tokens, E, K, renormalize, scale, topk_ids,
                       ids_is_i64, topk_weights);
  else if (experts <= 512)
    hipLaunchKernelGGL(router_topk_kernel<8>, g, b, 0, stream, logits, tokens, E, K, renormalize, scale, topk_ids,
                       ids_is_i64, topk_weights);
  else
    hipLaunchKernelGGL(router_topk_kernel<16>, g, b, 0, stream, logits, tokens, E, K, renormalize, scale, topk_ids,
                       ids_is_i64, topk_weights);
  return check_launch("router_topk");
}
