// moe_ext.cpp -- PyTorch-ROCm host extension `fused_cpp_amd._moe_C`.
//
// The C++ side of the Python operators: validates tensors, allocates the
// per-call workspace from the torch caching allocator on the current HIP
// stream, marshals device pointers into the C ABI of libfcmoe.so
// (include/fcmoe.h) and maps its error codes to RuntimeError. It plays the
// role of the reference's pybind modules `_moe_C` (csrc/moe/module.cpp:10-264)
// and `_C`'s i8gemm bindings (csrc/module.cpp:220-233); the GIL is released
// around every launch as there (module.cpp:206-220).
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <thread>
#include <unordered_map>
#include <string>
#include <tuple>

#include "../../include/fcmoe.h"

namespace {

constexpr int64_t kBackendId = 950;
const char* kBackendName = "gfx950_mfma";

hipStream_t current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == FCMOE_OK, what, " failed: ", fcmoe_last_error());
}

void check_device(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a ROCm (cuda) device tensor");
}

at::Tensor workspace(size_t bytes, const at::Tensor& like) {
  return at::empty({(int64_t)bytes}, like.options().dtype(at::kByte));
}

int activation_code(const std::string& name) {
  if (name == "silu") return FCMOE_ACT_SILU;
  if (name == "gelu") return FCMOE_ACT_GELU;
  if (name == "swigluoai") return FCMOE_ACT_SWIGLUOAI;
  if (name == "silu_clamp10") return FCMOE_ACT_SILU_CLAMP10;
  TORCH_CHECK(false, "unsupported MoE activation: ", name);
}

at::Tensor pack(const at::Tensor& w, int n_groups) {
  // w: [E, N, K] int8 or bf16 on device.
  const int eb = w.scalar_type() == at::kChar ? 1 : 2;
  const int64_t e = w.size(0), n = w.size(1), k = w.size(2);
  const int64_t per = fcmoe_packed_expert_bytes(eb, n, k, n_groups);
  TORCH_CHECK(per > 0, "invalid weight shape for packing");
  at::Tensor dst = at::empty({e, per}, w.options().dtype(at::kChar));
  check_rc(fcmoe_pack_experts(w.data_ptr(), eb, e, n, k, n_groups, dst.data_ptr(), current_stream()), "pack");
  return dst;
}

// Packs source experts `w` ([e, n, k] int8 or bf16, host or device) into rows
// [first, first + e) of `dst` ([E, per] int8 on the device). Host experts are
// staged through the device a chunk at a time (at most 256 MB and 1/16 of
// the source, at least one expert), so the device never holds a full second
// copy of them.
void pack_into(at::Tensor& dst, int64_t first, const at::Tensor& w, int n_groups) {
  const int eb = w.scalar_type() == at::kChar ? 1 : 2;
  const int64_t e = w.size(0), n = w.size(1), k = w.size(2);
  const int64_t per = dst.size(1);
  TORCH_CHECK(per == fcmoe_packed_expert_bytes(eb, n, k, n_groups), "packed expert size mismatch");
  const int64_t expert_bytes = n * k * eb;
  const int64_t stage_bytes = std::min<int64_t>(int64_t(256) << 20, e * expert_bytes / 16);
  const int64_t chunk = w.is_cuda() ? e : std::max<int64_t>(1, stage_bytes / std::max<int64_t>(expert_bytes, 1));
  for (int64_t i = 0; i < e; i += chunk) {
    const int64_t m = std::min(chunk, e - i);
    at::Tensor src = w.slice(0, i, i + m);
    src = src.is_cuda() ? src.contiguous() : src.to(dst.device()).contiguous();
    check_rc(fcmoe_pack_experts(src.data_ptr(), eb, m, n, k, n_groups, (int8_t*)dst.data_ptr() + (first + i) * per,
                                current_stream()),
             "pack");
  }
}

// Routed experts [E, n, k] plus one shared expert [n, k] packed as experts
// 0..E-1 and E of one buffer, without concatenating the sources first: the
// routed+shared prepare of src/fused_cpp/moe/bf16_tiled.py:541-570 (native
// fused_moe_bf16_tiled.cpp:6276-6288), which packs "without a full source copy".
at::Tensor pack_routed_shared(const at::Tensor& routed, const at::Tensor& shared, int n_groups,
                              const at::Device& dev) {
  TORCH_CHECK(routed.dim() == 3 && routed.size(0) > 0, "routed weights must be [E, N, K] with E > 0");
  at::Tensor sh = shared.dim() == 3 ? shared.squeeze(0) : shared;
  TORCH_CHECK(sh.dim() == 2 && sh.size(0) == routed.size(1) && sh.size(1) == routed.size(2),
              "the shared expert must match one routed expert's shape");
  TORCH_CHECK(sh.scalar_type() == routed.scalar_type(), "routed and shared weights must share a dtype");
  const int eb = routed.scalar_type() == at::kChar ? 1 : 2;
  const int64_t e = routed.size(0);
  const int64_t per = fcmoe_packed_expert_bytes(eb, routed.size(1), routed.size(2), n_groups);
  TORCH_CHECK(per > 0, "invalid weight shape for packing");
  at::Tensor dst = at::empty({e + 1, per}, at::TensorOptions().dtype(at::kChar).device(dev));
  pack_into(dst, 0, routed, n_groups);
  pack_into(dst, e, sh.unsqueeze(0), n_groups);
  return dst;
}

at::Device target_device(const at::Tensor& t) {
  if (t.is_cuda()) return t.device();
  return at::Device(at::kCUDA, c10::hip::current_device());
}

using W8A8Tuple =
    std::tuple<at::Tensor, int64_t, int64_t, at::Tensor, at::Tensor, int64_t, int64_t, at::Tensor, int64_t, int64_t>;

// Packs per-channel int8 experts plus fp32 scales. `what` names the path in
// errors; W8A8 requires H, F % 16 (csrc/moe/arm/i8mm_w8a8/kernels.cpp:55),
// W8A16 requires F % 8 (fused_moe_bf16_tiled.cpp:5035).
W8A8Tuple pack_int8_experts(at::Tensor w13, at::Tensor s13, at::Tensor w2, at::Tensor s2, const char* what,
                            bool w8a16) {
  check_device(w13, "w13_weight");
  check_device(w2, "w2_weight");
  TORCH_CHECK(w13.scalar_type() == at::kChar && w2.scalar_type() == at::kChar, what,
              " weights must have dtype torch.int8");
  TORCH_CHECK(w13.dim() == 3 && w2.dim() == 3, what, " weights must be [E, 2F, H] and [E, H, F]");
  TORCH_CHECK(w13.size(0) > 0 && w13.size(0) == w2.size(0), what, " expert counts must match and be positive");
  TORCH_CHECK(w13.size(1) % 2 == 0, what, " W13 output dimension must be even");
  const int64_t e = w13.size(0), f = w13.size(1) / 2, h = w13.size(2);
  TORCH_CHECK(w2.size(1) == h && w2.size(2) == f, what, " W2 shape mismatch");
  if (w8a16) {
    TORCH_CHECK(f % 8 == 0, "W8A16 fused W13 requires F % 8 == 0, got ", f);
  } else {
    TORCH_CHECK(h % 16 == 0 && f % 16 == 0, what, " requires H and F to be multiples of 16");
  }
  TORCH_CHECK(s13.scalar_type() == at::kFloat && s2.scalar_type() == at::kFloat, what, " scales must be float32");
  TORCH_CHECK(s13.numel() == e * 2 * f, what, " W13 scales must contain one value per output channel");
  TORCH_CHECK(s2.numel() == e * h, what, " W2 scales must contain one value per output channel");
  at::Tensor p13 = pack(w13.contiguous(), 2);
  at::Tensor p2 = pack(w2.contiguous(), 1);
  return {p13, h, 2 * f, s13.to(w13.device()).reshape({e, 2 * f}).contiguous(), p2, f, h,
          s2.to(w13.device()).reshape({e, h}).contiguous(), kBackendId, 16};
}

// Routed + shared checkpoint int8 experts (W8A8: bf16_tiled.py:573-609;
// W8A16: bf16_tiled.py:541-570): the shared expert is packed as expert E
// straight into the routed experts' buffer; only the fp32 scales (one value
// per channel) are concatenated.
W8A8Tuple int8_prepare_routed_shared(at::Tensor rw13, at::Tensor rs13, at::Tensor rw2, at::Tensor rs2,
                                     at::Tensor sw13, at::Tensor ss13, at::Tensor sw2, at::Tensor ss2, bool w8a16) {
  const char* what = w8a16 ? "W8A16" : "W8A8";
  TORCH_CHECK(rw13.scalar_type() == at::kChar && rw2.scalar_type() == at::kChar, what,
              " weights must have dtype torch.int8");
  TORCH_CHECK(rw13.dim() == 3 && rw2.dim() == 3, what, " weights must be [E, 2F, H] and [E, H, F]");
  TORCH_CHECK(rw13.size(0) > 0 && rw13.size(0) == rw2.size(0), what, " expert counts must match and be positive");
  TORCH_CHECK(rw13.size(1) % 2 == 0, what, " W13 output dimension must be even");
  const int64_t e = rw13.size(0), f = rw13.size(1) / 2, h = rw13.size(2);
  TORCH_CHECK(rw2.size(1) == h && rw2.size(2) == f, what, " W2 shape mismatch");
  if (w8a16) {
    TORCH_CHECK(f % 8 == 0, "W8A16 fused W13 requires F % 8 == 0, got ", f);
  } else {
    TORCH_CHECK(h % 16 == 0 && f % 16 == 0, what, " requires H and F to be multiples of 16");
  }
  TORCH_CHECK(rs13.numel() == e * 2 * f && ss13.numel() == 2 * f, what,
              " W13 scales must contain one value per output channel");
  TORCH_CHECK(rs2.numel() == e * h && ss2.numel() == h, what, " W2 scales must contain one value per output channel");
  const at::Device dev = target_device(rw13);
  at::Tensor p13 = pack_routed_shared(rw13, sw13, 2, dev);
  at::Tensor p2 = pack_routed_shared(rw2, sw2, 1, dev);
  auto f32 = [&](const at::Tensor& t, int64_t rows, int64_t cols) {
    return t.to(dev, at::kFloat).reshape({rows, cols});
  };
  at::Tensor s13 = at::cat({f32(rs13, e, 2 * f), f32(ss13, 1, 2 * f)}, 0).contiguous();
  at::Tensor s2 = at::cat({f32(rs2, e, h), f32(ss2, 1, h)}, 0).contiguous();
  return {p13, h, 2 * f, s13, p2, f, h, s2, kBackendId, 16};
}

// Packs checkpoint int8 experts (csrc/moe/arm/i8mm_w8a8/kernels.cpp:424-444).
W8A8Tuple w8a8_prepare_quantized(at::Tensor w13, at::Tensor s13, at::Tensor w2, at::Tensor s2) {
  return pack_int8_experts(w13, s13, w2, s2, "W8A8", false);
}

// W8A16 checkpoint packing (fused_moe_bf16_tiled.cpp:5012-5112): the same
// per-channel int8 + fp32 scale layout as W8A8.
W8A8Tuple w8a16_prepare_quantized(at::Tensor w13, at::Tensor s13, at::Tensor w2, at::Tensor s2) {
  return pack_int8_experts(w13, s13, w2, s2, "W8A16", true);
}

// Quantise bf16 experts per output channel on the GPU, then pack
// (csrc/moe/arm/i8mm_w8a8/kernels.cpp:446-461).
W8A8Tuple w8a8_prepare(at::Tensor w13, at::Tensor w2) {
  check_device(w13, "w13_weight");
  check_device(w2, "w2_weight");
  TORCH_CHECK(w13.scalar_type() == at::kBFloat16 && w2.scalar_type() == at::kBFloat16,
              "W8A8 source weights must have dtype torch.bfloat16");
  TORCH_CHECK(w13.dim() == 3 && w2.dim() == 3, "W8A8 weights must be [E, 2F, H] and [E, H, F]");
  auto quant = [](const at::Tensor& src) {
    at::Tensor s = src.contiguous();
    const int64_t cols = s.size(-1);
    const int64_t rows = s.numel() / cols;
    at::Tensor q = at::empty(s.sizes(), s.options().dtype(at::kChar));
    at::Tensor sc = at::empty({s.size(0), s.size(1)}, s.options().dtype(at::kFloat));
    check_rc(fcmoe_quantize_weight_rows((const uint16_t*)s.data_ptr(), rows, cols, (int8_t*)q.data_ptr(),
                                        sc.data_ptr<float>(), current_stream()),
             "quantize_weight_rows");
    return std::make_pair(q, sc);
  };
  auto [q13, s13] = quant(w13);
  auto [q2, s2] = quant(w2);
  return w8a8_prepare_quantized(q13, s13, q2, s2);
}

// W8A16 prepare from bf16 (fused_moe_bf16_tiled.cpp:6211-6266,
// quantize_pack_expert_weight_per_channel :4947-4976): the same per-channel
// quantisation as W8A8 (scale = max|w| / 127, or 1; q = nearbyint(w / scale)
// clamped to +-127).
W8A8Tuple w8a16_prepare(at::Tensor w13, at::Tensor w2) {
  check_device(w13, "w13_weight");
  check_device(w2, "w2_weight");
  TORCH_CHECK(w13.scalar_type() == at::kBFloat16 && w2.scalar_type() == at::kBFloat16,
              "W8A16 source weights must be torch.bfloat16");
  TORCH_CHECK(w13.dim() == 3 && w2.dim() == 3, "W8A16 weights must be [E, 2F, H] and [E, H, F]");
  auto quant = [](const at::Tensor& src) {
    at::Tensor s = src.contiguous();
    const int64_t cols = s.size(-1);
    const int64_t rows = s.numel() / cols;
    at::Tensor q = at::empty(s.sizes(), s.options().dtype(at::kChar));
    at::Tensor sc = at::empty({s.size(0), s.size(1)}, s.options().dtype(at::kFloat));
    check_rc(fcmoe_quantize_weight_rows((const uint16_t*)s.data_ptr(), rows, cols, (int8_t*)q.data_ptr(),
                                        sc.data_ptr<float>(), current_stream()),
             "quantize_weight_rows");
    return std::make_pair(q, sc);
  };
  auto [q13, s13] = quant(w13);
  auto [q2, s2] = quant(w2);
  return w8a16_prepare_quantized(q13, s13, q2, s2);
}

fcmoe_moe_args base_args(const at::Tensor& input, const at::Tensor& topk_weights, const at::Tensor& topk_ids,
                         int64_t experts, int64_t shared_id, double routed_scale, int64_t global_num_experts,
                         const at::Tensor& out) {
  fcmoe_moe_args a{};
  a.x = (const uint16_t*)input.data_ptr();
  a.tokens = input.size(0);
  a.hidden = input.size(1);
  a.top_k = topk_ids.defined() ? topk_ids.size(1) : 0;
  a.topk_ids = a.top_k > 0 ? topk_ids.data_ptr() : nullptr;
  a.ids_is_i64 = (topk_ids.defined() && topk_ids.scalar_type() == at::kLong) ? 1 : 0;
  a.topk_weights = a.top_k > 0 ? topk_weights.data_ptr<float>() : nullptr;
  a.experts = experts;
  a.valid_experts = global_num_experts > 0 ? global_num_experts : experts;
  a.shared_expert_id = shared_id;
  a.routed_scaling = (float)routed_scale;
  a.out = (uint16_t*)out.data_ptr();
  return a;
}

void check_routing(const at::Tensor& input, const at::Tensor& topk_weights, const at::Tensor& topk_ids) {
  check_device(input, "input");
  TORCH_CHECK(input.scalar_type() == at::kBFloat16 && input.dim() == 2 && input.is_contiguous(),
              "input must be a contiguous bf16 [tokens, hidden] tensor");
  if (!topk_ids.defined()) return;
  check_device(topk_ids, "topk_ids");
  check_device(topk_weights, "topk_weights");
  TORCH_CHECK(topk_ids.dim() == 2 && topk_weights.sizes() == topk_ids.sizes(),
              "topk tensors must be matching [tokens, top_k]");
  TORCH_CHECK(topk_ids.size(0) == input.size(0), "topk token dimension must match input");
  TORCH_CHECK(topk_ids.scalar_type() == at::kLong || topk_ids.scalar_type() == at::kInt,
              "topk_ids must be int32 or int64");
  TORCH_CHECK(topk_weights.scalar_type() == at::kFloat, "topk_weights must be float32");
  TORCH_CHECK(topk_ids.is_contiguous() && topk_weights.is_contiguous(), "topk tensors must be contiguous");
}

at::Tensor output_for(const at::Tensor& input, c10::optional<at::Tensor> out) {
  if (!out.has_value()) return at::empty_like(input);
  at::Tensor o = *out;
  TORCH_CHECK(o.device() == input.device() && o.scalar_type() == at::kBFloat16 && o.sizes() == input.sizes() &&
                  o.is_contiguous(),
              "out must be contiguous bf16 with the input shape on the input device");
  TORCH_CHECK(!o.requires_grad(), "out with requires_grad=True is not supported");
  return o;
}

// The synchronous invalid-id error of the reference (kernels.cpp:586 raises
// before computing). The route launch (the first of a forward) writes the
// count of ids outside the valid range; the host must see it before the call
// returns. Reading it from device memory (`.item()`) would wait for the whole
// forward, so the host could not enqueue the next call while this one runs.
// Instead the count goes to a per-thread, per-device slot of coherent pinned
// host memory, which the host polls: the call returns as soon as the route
// launch has finished, the rest of the forward still running on the stream.
// Under graph capture (nothing runs) and for empty batches (no route launch)
// the device tensor is used and read as before.
constexpr int32_t kPendingCount = INT32_MIN;

int32_t* pinned_count_slot() {
  thread_local std::unordered_map<int, int32_t*> slots;  // held until the thread ends (one 64-byte block each)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  int32_t*& slot = slots[dev];
  if (!slot) {
    void* p = nullptr;
    if (hipHostMalloc(&p, 64, hipHostMallocCoherent | hipHostMallocPortable) != hipSuccess) return nullptr;
    slot = (int32_t*)p;
  }
  return slot;
}

struct InvalidCheck {
  bool validate = false;
  int32_t* host = nullptr;  // pinned slot being polled (else: device tensor)
  at::Tensor dev;

  // Sets args->invalid_count for one forward on the current stream.
  InvalidCheck(bool v, const at::Tensor& input, fcmoe_moe_args* a) : validate(v) {
    if (!validate) {
      a->invalid_count = nullptr;
      return;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(current_stream(), &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    if (!capturing && input.size(0) > 0) host = pinned_count_slot();
    if (host) {
      __atomic_store_n(host, kPendingCount, __ATOMIC_RELEASE);
      void* dp = nullptr;
      TORCH_CHECK(hipHostGetDevicePointer(&dp, host, 0) == hipSuccess, "pinned invalid-id count not mapped");
      a->invalid_count = (int32_t*)dp;
    } else {
      dev = at::zeros({1}, input.options().dtype(at::kInt));
      a->invalid_count = dev.data_ptr<int32_t>();
    }
  }

  // A forward that failed part-way may still have its route launch queued:
  // let the stream drain before the slot can be reused by the next call.
  void check_rc(int rc, const char* what) {
    if (rc != FCMOE_OK && host) (void)hipStreamSynchronize(current_stream());
    ::check_rc(rc, what);
  }

  // After the forward was enqueued: raise if any id was out of range.
  void finish() {
    if (!validate) return;
    int32_t bad = 0;
    if (host) {
      pybind11::gil_scoped_release release;
      hipStream_t s = current_stream();
      // Spin on the slot alone for up to 1 ms (a runtime query per turn slowed
      // back-to-back one-token calls by ~3 us each), then also ask whether the
      // stream has drained (a forward whose route launch writes no count).
      const auto t0 = std::chrono::steady_clock::now();
      bool query = false;
      for (int i = 0;; ++i) {
        bad = __atomic_load_n(host, __ATOMIC_ACQUIRE);
        if (bad != kPendingCount) break;
#if defined(__x86_64__) || defined(__i386__)
        __builtin_ia32_pause();
#endif
        if (i % 256 != 255) continue;
        if (!query) {
          query = std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(1);
          if (!query) continue;
        }
        const hipError_t q = hipStreamQuery(s);
        if (q == hipSuccess) {  // the stream drained: the count is final (no route launch ran: no id checked)
          bad = __atomic_load_n(host, __ATOMIC_ACQUIRE);
          if (bad == kPendingCount) bad = 0;
          break;
        }
        TORCH_CHECK(q == hipErrorNotReady, "fused MoE: stream error while waiting for the id check: ",
                    hipGetErrorString(q));
        std::this_thread::yield();
      }
    } else {
      bad = dev.item<int32_t>();
    }
    TORCH_CHECK(bad == 0, "topk_ids out of range: ", bad, " id(s) outside the valid expert range");
  }
};

// W8A8 forward (csrc/moe/arm/i8mm_w8a8/kernels.cpp:463-694).
at::Tensor w8a8_forward(at::Tensor input, at::Tensor w13, int64_t w13_k, int64_t w13_n, at::Tensor s13,
                        at::Tensor w2, int64_t w2_k, int64_t w2_n, at::Tensor s2, at::Tensor topk_weights,
                        at::Tensor topk_ids, int64_t shared_id, double routed_scale, int64_t global_num_experts,
                        c10::optional<at::Tensor> out, bool validate_ids) {
  check_routing(input, topk_weights, topk_ids);
  check_device(w13, "w13_packed");
  TORCH_CHECK(input.size(1) == w13_k && w13_n == 2 * w2_k && w2_n == w13_k, "W8A8 expert dimensions mismatch");
  const int64_t e = w13.size(0);
  TORCH_CHECK(w2.size(0) == e && s13.sizes() == at::IntArrayRef({e, w13_n}) && s2.sizes() == at::IntArrayRef({e, w2_n}),
              "W8A8 packed weights/scales are invalid");
  TORCH_CHECK(w13.size(1) == fcmoe_packed_expert_bytes(1, w13_n, w13_k, 2) &&
                  w2.size(1) == fcmoe_packed_expert_bytes(1, w2_n, w2_k, 1),
              "W8A8 packed weight strides are invalid");
  at::Tensor output = output_for(input, out);
  fcmoe_moe_args a = base_args(input, topk_weights, topk_ids, e, shared_id, routed_scale, global_num_experts, output);
  a.inter = w2_k;
  a.w13 = w13.data_ptr();
  a.w2 = w2.data_ptr();
  a.w13_scale = s13.data_ptr<float>();
  a.w2_scale = s2.data_ptr<float>();
  a.activation = FCMOE_ACT_SILU_CLAMP10;
  InvalidCheck invalid(validate_ids, input, &a);
  at::Tensor ws = workspace(fcmoe_w8a8_workspace_bytes(&a), input);
  a.workspace = ws.data_ptr();
  a.workspace_bytes = ws.numel();
  {
    pybind11::gil_scoped_release release;
    invalid.check_rc(fcmoe_w8a8_forward(&a, current_stream()), "fused_moe_w8a8");
  }
  invalid.finish();
  return output;
}

using Bf16Tuple = std::tuple<at::Tensor, int64_t, int64_t, at::Tensor, int64_t, int64_t, int64_t, int64_t, std::string>;

// BF16 prepare (csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6125-6209).
Bf16Tuple bf16_prepare(at::Tensor w13, at::Tensor w2) {
  check_device(w13, "w13_weight");
  check_device(w2, "w2_weight");
  TORCH_CHECK(w13.scalar_type() == at::kBFloat16 && w2.scalar_type() == at::kBFloat16,
              "BF16 tiled fused MoE weights must be torch.bfloat16");
  TORCH_CHECK(w13.dim() == 3 && w2.dim() == 3, "weights must be [E, 2F, H] and [E, H, F]");
  TORCH_CHECK(w13.size(0) == w2.size(0) && w13.size(1) % 2 == 0 && w2.size(1) == w13.size(2) &&
                  w2.size(2) == w13.size(1) / 2,
              "w13/w2 shape mismatch");
  at::Tensor p13 = pack(w13.contiguous(), 2);
  at::Tensor p2 = pack(w2.contiguous(), 1);
  return {p13, w13.size(2), w13.size(1), p2, w2.size(2), w2.size(1), kBackendId, 16, std::string(kBackendName)};
}

// Routed + shared BF16 experts packed into one buffer (shared expert E)
// without concatenating the sources (bf16_tiled.py:573-609).
Bf16Tuple bf16_prepare_routed_shared(at::Tensor rw13, at::Tensor rw2, at::Tensor sw13, at::Tensor sw2) {
  TORCH_CHECK(rw13.scalar_type() == at::kBFloat16 && rw2.scalar_type() == at::kBFloat16,
              "BF16 tiled fused MoE weights must be torch.bfloat16");
  TORCH_CHECK(rw13.dim() == 3 && rw2.dim() == 3, "weights must be [E, 2F, H] and [E, H, F]");
  TORCH_CHECK(rw13.size(0) == rw2.size(0) && rw13.size(1) % 2 == 0 && rw2.size(1) == rw13.size(2) &&
                  rw2.size(2) == rw13.size(1) / 2,
              "w13/w2 shape mismatch");
  const at::Device dev = target_device(rw13);
  at::Tensor p13 = pack_routed_shared(rw13, sw13, 2, dev);
  at::Tensor p2 = pack_routed_shared(rw2, sw2, 1, dev);
  return {p13, rw13.size(2), rw13.size(1), p2, rw2.size(2), rw2.size(1), kBackendId, 16, std::string(kBackendName)};
}

at::Tensor bias_f32(c10::optional<at::Tensor> b, int64_t e, int64_t n, const at::Tensor& like) {
  if (!b.has_value() || !b->defined()) return at::Tensor();
  TORCH_CHECK(b->numel() == e * n, "bias must have shape [E, N]");
  return b->to(like.device(), at::kFloat).reshape({e, n}).contiguous();
}

// BF16 forward (csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6376-7218) and
// the shared MLP when topk_ids is undefined (:10307-10455).
at::Tensor bf16_forward(at::Tensor input, at::Tensor w13, int64_t w13_k, int64_t w13_n, at::Tensor w2, int64_t w2_k,
                        int64_t w2_n, c10::optional<at::Tensor> topk_weights_opt,
                        c10::optional<at::Tensor> topk_ids_opt, c10::optional<at::Tensor> w13_bias,
                        c10::optional<at::Tensor> w2_bias, std::string activation, int64_t global_num_experts,
                        bool skip_weighted, int64_t shared_id, double routed_scale, c10::optional<at::Tensor> out,
                        bool validate_ids) {
  at::Tensor topk_weights = topk_weights_opt.value_or(at::Tensor());
  at::Tensor topk_ids = topk_ids_opt.value_or(at::Tensor());
  check_routing(input, topk_weights, topk_ids);
  check_device(w13, "w13_packed");
  TORCH_CHECK(input.size(1) == w13_k && w13_n % 2 == 0 && w2_k == w13_n / 2 && w2_n == w13_k,
              "BF16 expert dimensions mismatch");
  const int64_t e = w13.size(0);
  TORCH_CHECK(w2.size(0) == e && w13.size(1) == fcmoe_packed_expert_bytes(2, w13_n, w13_k, 2) &&
                  w2.size(1) == fcmoe_packed_expert_bytes(2, w2_n, w2_k, 1),
              "BF16 packed weights are invalid");
  at::Tensor output = output_for(input, out);
  at::Tensor b13 = bias_f32(w13_bias, e, w13_n, input);
  at::Tensor b2 = bias_f32(w2_bias, e, w2_n, input);
  fcmoe_moe_args a = base_args(input, topk_weights, topk_ids, e, shared_id, routed_scale, global_num_experts, output);
  a.inter = w2_k;
  a.w13 = w13.data_ptr();
  a.w2 = w2.data_ptr();
  a.w13_bias = b13.defined() ? b13.data_ptr<float>() : nullptr;
  a.w2_bias = b2.defined() ? b2.data_ptr<float>() : nullptr;
  a.activation = activation_code(activation);
  a.skip_weighted = skip_weighted ? 1 : 0;
  InvalidCheck invalid(validate_ids, input, &a);
  at::Tensor ws = workspace(fcmoe_bf16_workspace_bytes(&a), input);
  a.workspace = ws.data_ptr();
  a.workspace_bytes = ws.numel();
  {
    pybind11::gil_scoped_release release;
    invalid.check_rc(fcmoe_bf16_forward(&a, current_stream()), "fused_moe_bf16");
  }
  invalid.finish();
  return output;
}

// W8A16 forward (bf16_tiled.py:1309-1373; native fused_moe_bf16_tiled.cpp
// W8A16 executor): int8 per-channel weights, bf16 activations, fp32 accumulate
// with the channel scale applied to the accumulator, bf16 intermediate.
at::Tensor w8a16_forward(at::Tensor input, at::Tensor w13, int64_t w13_k, int64_t w13_n, at::Tensor s13,
                         at::Tensor w2, int64_t w2_k, int64_t w2_n, at::Tensor s2, at::Tensor topk_weights,
                         at::Tensor topk_ids, std::string activation, int64_t global_num_experts, bool skip_weighted,
                         int64_t shared_id, double routed_scale, c10::optional<at::Tensor> out, bool validate_ids) {
  check_routing(input, topk_weights, topk_ids);
  check_device(w13, "w13_packed");
  TORCH_CHECK(input.size(1) == w13_k && w13_n == 2 * w2_k && w2_n == w13_k, "W8A16 expert dimensions mismatch");
  const int64_t e = w13.size(0);
  TORCH_CHECK(w2.size(0) == e && s13.sizes() == at::IntArrayRef({e, w13_n}) && s2.sizes() == at::IntArrayRef({e, w2_n}),
              "W8A16 packed weights/scales are invalid");
  TORCH_CHECK(w13.size(1) == fcmoe_packed_expert_bytes(1, w13_n, w13_k, 2) &&
                  w2.size(1) == fcmoe_packed_expert_bytes(1, w2_n, w2_k, 1),
              "W8A16 packed weight strides are invalid");
  at::Tensor output = output_for(input, out);
  fcmoe_moe_args a = base_args(input, topk_weights, topk_ids, e, shared_id, routed_scale, global_num_experts, output);
  a.inter = w2_k;
  a.w13 = w13.data_ptr();
  a.w2 = w2.data_ptr();
  a.w13_scale = s13.data_ptr<float>();
  a.w2_scale = s2.data_ptr<float>();
  a.activation = activation_code(activation);
  a.skip_weighted = skip_weighted ? 1 : 0;
  InvalidCheck invalid(validate_ids, input, &a);
  at::Tensor ws = workspace(fcmoe_w8a16_workspace_bytes(&a), input);
  a.workspace = ws.data_ptr();
  a.workspace_bytes = ws.numel();
  {
    pybind11::gil_scoped_release release;
    invalid.check_rc(fcmoe_w8a16_forward(&a, current_stream()), "fused_moe_w8a16");
  }
  invalid.finish();
  return output;
}

// i8gemm prepare (csrc/i8gemm.cpp:280-316): packed weight, fp32 [N] scales,
// K, N, Kp, Np, backend name.
std::tuple<at::Tensor, at::Tensor, int64_t, int64_t, int64_t, int64_t, std::string> i8gemm_prepare(
    at::Tensor weight, at::Tensor weight_scale) {
  check_device(weight, "weight");
  TORCH_CHECK(weight.dim() == 2, "i8gemm.prepare: weight must be 2D [N, K], got dim=", weight.dim());
  TORCH_CHECK(weight.scalar_type() == at::kChar, "i8gemm.prepare: weight dtype must be torch.int8");
  const int64_t n = weight.size(0), k = weight.size(1);
  TORCH_CHECK(n > 0 && k > 0, "i8gemm.prepare: N and K must be positive, got N=", n, " K=", k);
  at::Tensor scale = weight_scale.to(weight.device(), at::kFloat).reshape({-1});
  TORCH_CHECK(scale.numel() == 1 || scale.numel() == n, "i8gemm.prepare: weight_scale must be scalar or shape [N]");
  if (scale.numel() == 1) scale = scale.expand({n});
  at::Tensor packed = pack(weight.contiguous().unsqueeze(0), 1).reshape({-1});
  return {packed, scale.contiguous(), k, n, fcmoe_packed_expert_bytes(1, n, k, 1) / (((n + 15) / 16) * 16),
          ((n + 15) / 16) * 16, std::string(kBackendName)};
}

// i8gemm_dynamic_scaled_mm (csrc/i8gemm.cpp:318-452).
void i8gemm_dynamic_scaled_mm(at::Tensor output, at::Tensor input, at::Tensor packed_weight, at::Tensor weight_scale,
                              c10::optional<at::Tensor> bias, int64_t k, int64_t n) {
  check_device(input, "input");
  TORCH_CHECK(input.dim() == 2 && input.is_contiguous(), "i8gemm.dynamic_scaled_mm: input must be contiguous [M, K]");
  TORCH_CHECK(input.scalar_type() == at::kFloat || input.scalar_type() == at::kBFloat16,
              "i8gemm.dynamic_scaled_mm: input dtype must be float32/bfloat16");
  TORCH_CHECK(output.dim() == 2 && output.is_contiguous() && output.size(0) == input.size(0) && output.size(1) == n,
              "i8gemm.dynamic_scaled_mm: output shape must be [M, N]");
  TORCH_CHECK(output.scalar_type() == at::kFloat || output.scalar_type() == at::kBFloat16,
              "i8gemm.dynamic_scaled_mm: output dtype must be float32/bfloat16");
  TORCH_CHECK(input.size(1) == k, "i8gemm.dynamic_scaled_mm: input K mismatch");
  TORCH_CHECK(packed_weight.numel() == fcmoe_packed_expert_bytes(1, n, k, 1), "i8gemm: invalid packed_weight");
  TORCH_CHECK(weight_scale.numel() == n && weight_scale.scalar_type() == at::kFloat,
              "i8gemm.dynamic_scaled_mm: weight_scale must be contiguous float32 [N]");
  const int64_t m = input.size(0);
  if (m == 0) return;
  at::Tensor b;
  if (bias.has_value() && bias->defined()) {
    TORCH_CHECK(bias->dim() == 1 && bias->size(0) == n, "i8gemm.dynamic_scaled_mm: bias must be shape [", n, "]");
    b = bias->to(input.device(), at::kFloat).contiguous();
  }
  at::Tensor ws = workspace(fcmoe_i8gemm_workspace_bytes(m, k, n), input);
  pybind11::gil_scoped_release release;
  check_rc(fcmoe_i8gemm(input.data_ptr(), input.scalar_type() == at::kFloat ? 1 : 0, m, k, packed_weight.data_ptr(),
                        weight_scale.data_ptr<float>(), n, b.defined() ? b.data_ptr<float>() : nullptr,
                        output.data_ptr(), output.scalar_type() == at::kBFloat16 ? 1 : 0, ws.data_ptr(), ws.numel(),
                        current_stream()),
           "i8gemm");
}

// i8gemm_dynamic_scaled_mm_pair (csrc/i8gemm.cpp:453-570): one activation
// quantisation shared by two bf16-output GEMMs.
void i8gemm_dynamic_scaled_mm_pair(at::Tensor out1, at::Tensor out2, at::Tensor input, at::Tensor w1,
                                   at::Tensor s1, int64_t k, int64_t n1, at::Tensor w2, at::Tensor s2, int64_t n2) {
  check_device(input, "input");
  TORCH_CHECK(input.dim() == 2 && input.is_contiguous() && input.scalar_type() == at::kBFloat16 && input.size(1) == k,
              "i8gemm.dynamic_scaled_mm_pair: input must be contiguous BF16 [M, K]");
  const int64_t m = input.size(0);
  for (auto [o, w, sc, n, name] : {std::tuple<at::Tensor&, at::Tensor&, at::Tensor&, int64_t, const char*>{
                                       out1, w1, s1, n1, "first"},
                                   std::tuple<at::Tensor&, at::Tensor&, at::Tensor&, int64_t, const char*>{
                                       out2, w2, s2, n2, "second"}}) {
    TORCH_CHECK(o.scalar_type() == at::kBFloat16 && o.is_contiguous() && o.sizes() == at::IntArrayRef({m, n}), name,
                " output must be contiguous BF16 [M, N]");
    TORCH_CHECK(w.numel() == fcmoe_packed_expert_bytes(1, n, k, 1), name, " packed weight is invalid");
    TORCH_CHECK(sc.numel() == n && sc.scalar_type() == at::kFloat && sc.is_contiguous(), name,
                " scale must be contiguous float32 [N]");
  }
  if (m == 0) return;
  at::Tensor ws = workspace(fcmoe_i8gemm_pair_workspace_bytes(m, k, n1, n2), input);
  pybind11::gil_scoped_release release;
  check_rc(fcmoe_i8gemm_pair((const uint16_t*)input.data_ptr(), m, k, w1.data_ptr(), s1.data_ptr<float>(), n1,
                             w2.data_ptr(), s2.data_ptr<float>(), n2, (uint16_t*)out1.data_ptr(),
                             (uint16_t*)out2.data_ptr(), ws.data_ptr(), ws.numel(), current_stream()),
           "i8gemm_pair");
}

std::vector<std::string> available_backends() { return {kBackendName}; }

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "MI355X (gfx950) fused MoE host extension over libfcmoe";
  m.def("available_backends", &available_backends);
  m.def("abi_version", []() { return fcmoe_abi_version(); });
  m.def("fused_moe_w8a8_prepare_weights", &w8a8_prepare);
  m.def("fused_moe_w8a8_prepare_quantized_weights", &w8a8_prepare_quantized);
  m.def("fused_moe_w8a8_forward", &w8a8_forward);
  m.def("fused_moe_w8a16_prepare_weights", &w8a16_prepare);
  m.def("fused_moe_w8a16_prepare_quantized_weights", &w8a16_prepare_quantized);
  m.def("fused_moe_w8a16_forward", &w8a16_forward);
  m.def("fused_moe_bf16_prepare_weights", &bf16_prepare);
  m.def("fused_moe_bf16_prepare_routed_shared_weights", &bf16_prepare_routed_shared);
  m.def("fused_moe_int8_prepare_routed_shared_weights", &int8_prepare_routed_shared);
  m.def("fused_moe_bf16_forward", &bf16_forward);
  m.def("i8gemm_prepare", &i8gemm_prepare);
  m.def("i8gemm_dynamic_scaled_mm", &i8gemm_dynamic_scaled_mm);
  m.def("i8gemm_dynamic_scaled_mm_pair", &i8gemm_dynamic_scaled_mm_pair);
}
