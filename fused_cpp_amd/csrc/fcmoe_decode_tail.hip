// fcmoe_decode_tail.hip -- small-batch W8A8 decode in few launches. The
// decode head (below) does route, token-row quantisation and W13 for a
// one-token batch. The decode tail does the last three steps of the layer in
// one launch for a token or two:
//   requant: quantize_bf16_row of each route's intermediate row
//            (csrc/moe/arm/i8mm_w8a8/kernels.cpp:650-657, 211-228),
//   W2:      the int8 GEMM row with store_w2's scaling (kernels.cpp:248-257),
//   merge:   the ordered top-k FMA over the token's slots (kernels.cpp:674-688).
// At one token these are three launches of a few microseconds each around a
// 24 us weight stream; here they are one.
//
// Workgroup (tile, t) owns output channels 16 tile .. 16 tile + 15 of token t
// and has one wave per slot (top_k + shared), so the weight streams are as
// many as the unfused W2 launch's. A wave streams its slot expert's W2 tile
// through a ring and passes the route row through row 0 of
// v_mfma_i32_16x16x64_i8: per 64-byte K chunk each lane quantises one element
// of the row (with the row scale from the W13 epilogue's tile maxima), writes
// the byte to the wave's LDS ring, and lanes 16 g .. 16 g + 15 read bytes
// 16 g .. 16 g + 15 back as their A fragment (every row of the fragment holds
// the route row; only row 0 of the result is used). The slots' values meet in
// LDS and wave 0 merges them in slot order.
//
// The arithmetic is that of requant_kernel, the W2 epilogue and combine_kernel
// value for value, so the output is the same bit for bit, and so are the
// q2 / s2row / route_out views the unfused path leaves (every wave writes its
// channels of route_out; the waves of channel tile 0 also write their rows of
// q2 and the row scales).

#include "fcmoe_device.h"
#include "fcmoe_gemm_common.h"
#include "fcmoe_internal.h"
#include "fcmoe_quant_row.h"

namespace fcmoe {
namespace {

constexpr int kRing = 12;   // weight / y chunks per wave ring (issue runs kRing - 1 ahead)
constexpr int kQAhead = 2;  // chunks quantised ahead of the MFMA
constexpr int kQRing = 4;   // per-wave LDS ring of quantised 64-byte chunks
constexpr int kHeadEarly = 8;  // head: weight chunks issued before the token row is quantised (246 VGPRs: two waves per SIMD)

__global__ __launch_bounds__(kDecodeTailSlots * kWave) void decode_tail_kernel(DecodeTailArgs a) {
  __shared__ float s_val[kDecodeTailSlots][16];
  __shared__ float s_wt[kDecodeTailSlots];
  __shared__ int s_ok[kDecodeTailSlots];
  __shared__ __attribute__((aligned(16))) int8_t s_q[kDecodeTailSlots][kQRing][kWave];

  const int lane = threadIdx.x % kWave;
  const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int tile = blockIdx.x;
  const int t = blockIdx.y;
  const int col = lane % 16;
  const int64_t ch = (int64_t)tile * 16 + col;
  const bool cvalid = ch < a.hidden;
  const int64_t r = (int64_t)t * a.kt + slot;
  // the route's position and expert id, loaded together (the id is valid
  // whenever the position is)
  const int pos = a.route_pos[r];  // -1: the id was invalid and the route is dropped
  // (with top_k = 0 there are no ids: the only slot is the shared expert)
  const int64_t idx = (int64_t)t * a.top_k + (slot < a.top_k ? slot : 0);
  const int eid = a.top_k == 0 ? 0
                  : a.ids_is_i64 ? (int)((const int64_t*)a.ids)[idx]
                                 : ((const int32_t*)a.ids)[idx];
  if (pos >= 0) {
    const int e = slot < a.top_k ? eid : a.shared_id;
    const int kc = (int)a.k_chunks;
    const uint8_t* wb = (const uint8_t*)a.w + (int64_t)e * a.w_expert_bytes + (int64_t)tile * kc * 1024;
    const uint32_t* yw = (const uint32_t*)(a.y + (int64_t)pos * a.ldy);  // 32-bit words: two bf16 each
    v4i bq[kRing];
    uint32_t yq[kRing];
    // Chunks past the last re-load the last one (never consumed). y is read
    // as the 32-bit word holding this lane's bf16: a 16-bit value in the ring
    // makes the compiler re-extend it at the loop's back edge after waiting
    // for every load.
    auto issue = [&](int c, auto slot_c) {
      constexpr int b = decltype(slot_c)::value;
      const int cc = c < kc ? c : kc - 1;
      bq[b] = __builtin_nontemporal_load((const v4i*)(wb + (int64_t)cc * 1024) + lane);
      yq[b] = yw[(cc * 64 + lane) / 2];
    };
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (issue(S, std::integral_constant<int, S>{}), ...);
    }(std::make_integer_sequence<int, kRing - 1>{});

    // requant_kernel's row scale: the max of the row's tile maxima (clamped
    // indices re-read an entry, which leaves the max unchanged)
    const float* rp = a.rowpart + (int64_t)pos * a.parts;
    const int64_t i0 = lane < a.parts ? lane : a.parts - 1;
    const int64_t i1 = lane + kWave < a.parts ? lane + kWave : a.parts - 1;
    const float m = wave_max(fmaxf(rp[i0], rp[i1]));
    const float scale = m > 0.0f ? m / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    const float cs = a.scale_col[(int64_t)e * a.hidden + (cvalid ? ch : 0)];

    // per 64-byte chunk: each lane quantises one element (columns past I are
    // the requant's zero padding) into this wave's LDS ring; lanes 16 g ..
    // 16 g + 15 read bytes 16 g .. 16 g + 15 back as their A fragment
    int8_t(*q)[kWave] = s_q[slot];
    auto quantise = [&](int c, auto slot_c) {
      constexpr int b = decltype(slot_c)::value;
      const int k = c * 64 + lane;
      const uint32_t bits = (lane & 1) ? (yq[b] & 0xffff0000u) : (yq[b] << 16);  // bf16 -> fp32
      const float yv = k < a.inter ? __uint_as_float(bits) : 0.0f;
      q[c % kQRing][lane] = quant_value(yv, scale, inv, 0);
    };
    auto read_a = [&](int c) -> v4i { return *(const v4i*)(&q[c % kQRing][16 * (lane / 16)]); };
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (quantise(S, std::integral_constant<int, S>{}), ...);
    }(std::make_integer_sequence<int, kQAhead>{});
    v4i a_cur = read_a(0);
    v4i acc = v4i{0, 0, 0, 0};
    auto body = [&](int c, auto b_c) {
      constexpr int b = decltype(b_c)::value;
      issue(c + kRing - 1, std::integral_constant<int, (b + kRing - 1) % kRing>{});
      quantise(c + kQAhead, std::integral_constant<int, (b + kQAhead) % kRing>{});  // past the end: never read
      const v4i a_next = read_a(c + 1);
      acc = mfma(a_cur, bq[b % kRing], acc);
      a_cur = a_next;
    };
    int c0 = 0;
    for (; c0 + kRing <= kc; c0 += kRing) {
      [&]<int... S>(std::integer_sequence<int, S...>) {
        (body(c0 + S, std::integral_constant<int, S>{}), ...);
      }(std::make_integer_sequence<int, kRing>{});
    }
    [&]<int... S>(std::integer_sequence<int, S...>) {
      ((c0 + S < kc ? body(c0 + S, std::integral_constant<int, S>{}) : void()), ...);
    }(std::make_integer_sequence<int, kRing - 1>{});

    // store_w2 (kernels.cpp:248-257): output row 0 is lanes 0..15, register 0
    const float val = (float)acc[0] * (scale * cs);
    if (lane < 16) {
      s_val[slot][col] = val;
      if (cvalid) a.route_out[r * a.hidden + ch] = val;
    }
    if (lane == 0) {
      s_wt[slot] = a.route_weight[r];
      s_ok[slot] = 1;
    }
    // the q2 / s2row views (channel tile 0 only): the row quantised again
    if (tile == 0) {
      if (lane == 0) a.s2row[pos] = scale;
      for (int64_t k = lane; k < a.ldq; k += kWave) {
        const float yv = k < a.inter ? bf16_to_f32(a.y[(int64_t)pos * a.ldy + k]) : 0.0f;
        a.q2[(int64_t)pos * a.ldq + k] = quant_value(yv, scale, inv, 0);
      }
    }
  } else if (lane == 0) {
    s_ok[slot] = 0;
  }
  __syncthreads();
  // the ordered top-k merge (kernels.cpp:674-688): slots in order, dropped ones left out
  if (slot == 0 && lane < 16 && cvalid) {
    float merged = 0.0f;
    for (int s = 0; s < a.kt; ++s)
      if (s_ok[s]) merged = __builtin_fmaf(s_val[s][col], s_wt[s], merged);
    a.out[(int64_t)t * a.hidden + ch] = f32_to_bf16(merged);
  }
}


// ---- one-token head: route + token-row quantisation + W13 in one launch.
//
// Workgroup (j, s) is one wave: gate/up channel tile pair j of slot s of the
// single token. It reads the token's ids, derives its route's sorted position
// (routes ordered by expert, then by slot: the ascending flat route order of
// kernels.cpp:583-592) with a ballot, quantises the token row into LDS
// (quantize_bf16_row, kernels.cpp:211-228) and streams its expert's gate and
// up tiles through a ring, the row in row 0 of the MFMA as in the tail. The
// epilogue is the W13 one (w13_epilogue, kernels.cpp:230-246: clamped SwiGLU
// with the FEXPA exp, bf16 y and the per-(row, gate tile) max of |y|).
// Workgroups j = 0 write the route metadata the tail and the stage views read
// (route_pos, route_weight, sorted_routes, row_token); (0, 0) writes the
// invalid-id count.
template <int CAP>
__global__ __launch_bounds__(kWave) void decode_head_kernel(DecodeHeadArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t s_x[kDecodeHeadMaxK];
  const int lane = threadIdx.x;
  const int j = blockIdx.x;
  const int s = blockIdx.y;

  // the token row: CAP 16-byte units per lane, in flight with the ids
  const int64_t units = a.hidden / 8;
  const uint4* xp = (const uint4*)a.x;
  uint4 xv[CAP];
#pragma unroll
  for (int u = 0; u < CAP; ++u) {
    // unconditional loads (a conditional one would be waited for alone):
    // units past the row re-read its last unit, which leaves the max
    // unchanged; the quantised row holds zeros there
    const int64_t i = lane + (int64_t)u * kWave;
    xv[u] = xp[i < units ? i : units - 1];
  }
  // the token's slots: expert, validity (route_expert) and combined weight (route_weight_of)
  int e_l = 0;
  bool ok_l = false;
  float w_l = 0.0f;
  {
    // unconditional loads, results selected (top_k = 0: no ids, only the shared slot)
    const int li = lane < a.top_k ? lane : 0;
    const int64_t e = a.top_k == 0 ? 0
                      : a.ids_is_i64 ? ((const int64_t*)a.ids)[li]
                                     : (int64_t)((const int32_t*)a.ids)[li];
    float w = a.topk_w && a.top_k > 0 ? a.topk_w[li] : 1.0f;
    if (a.scale_routed) w = w * a.scale;
    if (lane < a.top_k) {
      ok_l = e >= 0 && e < a.valid_experts;
      e_l = ok_l ? (int)e : 0;
      w_l = w;
    } else if (lane < a.kt) {
      e_l = a.shared_id;
      ok_l = true;
      w_l = 1.0f;
    }
  }
  const int e_s = __builtin_amdgcn_readlane(e_l, s);
  const bool ok_s = __builtin_amdgcn_readlane((int)ok_l, s) != 0;
  const int pos = __popcll(__ballot(ok_l && (e_l < e_s || (e_l == e_s && lane < s))));
  const int n_invalid = __popcll(__ballot(lane < a.top_k && !ok_l));  // all lanes vote
  if (j == 0 && lane == 0) {
    a.route_pos[s] = ok_s ? pos : -1;
    a.route_weight[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w_l), s));
    if (ok_s) {
      a.sorted_routes[pos] = s;
      a.row_token[pos] = 0;
    }
    if (s == 0) store_count(a.invalid, n_invalid);
  }
  if (!ok_s) return;

  // gate tile j and up tile n_tiles + j of expert e_s (packed [group][tile][chunk][1 KB]);
  // the ring's first chunks go out before the row is quantised
  const int kc = (int)a.k_chunks;
  const uint8_t* wg = (const uint8_t*)a.w + (int64_t)e_s * a.w_expert_bytes + (int64_t)j * kc * 1024;
  const uint8_t* wu = wg + (int64_t)a.n_tiles * kc * 1024;
  v4i bg[kRing], bu[kRing];
  auto issue = [&](int c, auto slot_c) {
    constexpr int b = decltype(slot_c)::value;
    const int cc = c < kc ? c : kc - 1;  // past the end: re-read, never consumed
    bg[b] = __builtin_nontemporal_load((const v4i*)(wg + (int64_t)cc * 1024) + lane);
    bu[b] = __builtin_nontemporal_load((const v4i*)(wu + (int64_t)cc * 1024) + lane);
  };
  // the first kHeadEarly chunks before the row is quantised, the rest after
  // (all at once, the row's registers and the ring would not fit two waves
  // per SIMD)
  [&]<int... S>(std::integer_sequence<int, S...>) {
    (issue(S, std::integral_constant<int, S>{}), ...);
  }(std::make_integer_sequence<int, kHeadEarly>{});
  // quantize_bf16_row: scale = max|x| / 127, q = round(x / scale) half away
  float m = 0.0f;
#pragma unroll
  for (int u = 0; u < CAP; ++u) {
    const uint32_t w[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      m = fmaxf(m, fabsf(__uint_as_float(w[k] << 16)));
      m = fmaxf(m, fabsf(__uint_as_float(w[k] & 0xffff0000u)));
    }
  }
  m = wave_max(m);
  const float xs = m > 0.0f ? m / 127.0f : 1.0f;
  const float xinv = 1.0f / xs;
  if (j == 0 && s == 0 && lane == 0) *a.xs = xs;
#pragma unroll
  for (int u = 0; u < CAP; ++u) {
    const int64_t i = lane + (int64_t)u * kWave;
    if (i * 8 < a.k_chunks * 64) {
      const uint32_t w[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t qa = (uint8_t)quant_value(__uint_as_float(w[k] << 16), xs, xinv, 0);
        const uint32_t qb = (uint8_t)quant_value(__uint_as_float(w[k] & 0xffff0000u), xs, xinv, 0);
        const uint32_t pair = qa | (qb << 8);
        if (k < 2)
          lo |= pair << (16 * k);
        else
          hi |= pair << (16 * (k - 2));
      }
      *(uint2*)(&s_x[i * 8]) = i < units ? make_uint2(lo, hi) : make_uint2(0, 0);  // K padding: zeros
    }
  }
  __syncthreads();
  [&]<int... S>(std::integer_sequence<int, S...>) {
    (issue(kHeadEarly + S, std::integral_constant<int, kHeadEarly + S>{}), ...);
  }(std::make_integer_sequence<int, kRing - 1 - kHeadEarly>{});

  v4i acc_g = v4i{0, 0, 0, 0}, acc_u = v4i{0, 0, 0, 0};
  const int a_off = 16 * (lane / 16);
  auto body = [&](int c, auto b_c) {
    constexpr int b = decltype(b_c)::value;
    issue(c + kRing - 1, std::integral_constant<int, (b + kRing - 1) % kRing>{});
    const v4i av = *(const v4i*)(&s_x[c * 64 + a_off]);
    acc_g = mfma(av, bg[b % kRing], acc_g);
    acc_u = mfma(av, bu[b % kRing], acc_u);
  };
  int c0 = 0;
  for (; c0 + kRing <= kc; c0 += kRing) {
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (body(c0 + S, std::integral_constant<int, S>{}), ...);
    }(std::make_integer_sequence<int, kRing>{});
  }
  [&]<int... S>(std::integer_sequence<int, S...>) {
    ((c0 + S < kc ? body(c0 + S, std::integral_constant<int, S>{}) : void()), ...);
  }(std::make_integer_sequence<int, kRing - 1>{});

  // w13_epilogue on output row 0 (lanes 0..15, register 0); evaluated on every
  // lane so the FEXPA table read sees all lanes active
  const int col = lane % 16;
  const int64_t f = (int64_t)j * 16 + col;
  const bool fv = f < a.inter;
  const int64_t fc = fv ? f : 0;
  const float cg = a.scale_col[(int64_t)e_s * 2 * a.inter + fc];
  const float cu = a.scale_col[(int64_t)e_s * 2 * a.inter + a.inter + fc];
  float gate = (float)acc_g[0] * (xs * cg);
  float up = (float)acc_u[0] * (xs * cu);
  gate = fminf(gate, 10.0f);
  up = fmaxf(fminf(up, 10.0f), -10.0f);
  const float ex = fexpa_exp_neg_v(gate, fexpa_table_lane());
  const float y = (gate * up) / (ex + 1.0f);
  const uint16_t yb = f32_to_bf16(y);
  float ya = 0.0f;
  if (lane < 16 && fv) {
    a.y[(int64_t)pos * a.ldy + f] = yb;
    ya = fabsf(bf16_to_f32(yb));
  }
  const float amax = max16(ya);
  if (lane == 0) a.rowpart[(int64_t)pos * a.n_tiles + j] = amax;
}

}  // namespace

int decode_tail_launch(const DecodeTailArgs& a, hipStream_t stream) {
  if (a.tokens <= 0) return FCMOE_OK;
  if (a.kt <= 0 || a.kt > kDecodeTailSlots || a.parts > 2 * kWave || a.k_chunks <= 0 || a.ldq != a.k_chunks * 64 ||
      a.ldy < a.k_chunks * 64 || a.hidden <= 0 || a.tokens > 65535)
    return fail(FCMOE_EINVAL, "decode tail: shapes outside its domain");
  hipLaunchKernelGGL(decode_tail_kernel, dim3((unsigned)ceil_div(a.hidden, 16), (unsigned)a.tokens),
                     dim3(a.kt * kWave), 0, stream, a);
  return check_launch("decode_tail");
}

int decode_head_launch(const DecodeHeadArgs& a, hipStream_t stream) {
  const int64_t units = ceil_div(a.hidden / 8, kWave);  // x units per lane
  if (a.kt <= 0 || a.kt > kDecodeTailSlots || a.hidden % 8 || a.k_chunks * 64 > kDecodeHeadMaxK ||
      a.k_chunks * 64 < a.hidden || units > 16 || a.n_tiles <= 0)
    return fail(FCMOE_EINVAL, "decode head: shapes outside its domain");
  const dim3 grid((unsigned)a.n_tiles, (unsigned)a.kt), block(kWave);
  if (units <= 4)
    hipLaunchKernelGGL(decode_head_kernel<4>, grid, block, 0, stream, a);
  else if (units <= 8)
    hipLaunchKernelGGL(decode_head_kernel<8>, grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL(decode_head_kernel<16>, grid, block, 0, stream, a);
  return check_launch("decode_head");
}

}  // namespace fcmoe
