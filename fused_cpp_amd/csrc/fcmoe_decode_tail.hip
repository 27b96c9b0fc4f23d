// fcmoe_decode_tail.hip -- the last three steps of the W8A8 layer in one
// launch for decode batches of a token or two:
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
  const int pos = a.route_pos[r];  // -1: the id was invalid and the route is dropped
  if (pos >= 0) {
    const int64_t idx = (int64_t)t * a.top_k + slot;
    const int e = slot < a.top_k ? (a.ids_is_i64 ? (int)((const int64_t*)a.ids)[idx] : ((const int32_t*)a.ids)[idx])
                                 : a.shared_id;
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

}  // namespace fcmoe
