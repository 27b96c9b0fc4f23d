"""Host-side checks that need no GPU: the C ABI library loads and exports every
symbol declared in include/fcmoe.h, the Python surface mirrors the
reference's, and the wrappers' routing/validation logic (monkeypatched native
calls, as the reference's own tests do: tests/test_moe_w8a8.py:105-162)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent

# fused_cpp.moe.__all__ (src/fused_cpp/moe/__init__.py:67-126)
REFERENCE_MOE_ALL = {
    "ASYNC_MOE_EXECUTION_STRICT", "ASYNC_MOE_EXECUTION_TAIL_POOL", "ASYNC_MOE_FULL_EXPERT_RANGE",
    "ASYNC_MOE_PLACEMENT_FIXED", "ASYNC_MOE_PLACEMENT_TAIL_POOL", "ASYNC_MOE_PLAN_VERSION",
    "ASYNC_MOE_RESIZE_NONE", "ASYNC_MOE_STAGE_EXPERT", "AsyncMoEPlanV2", "DEFAULT_MOE_COST_CACHE_DIR",
    "MoePlannerRuntime", "PreparedBF16TiledFusedMoEWeights", "PreparedBF16TiledRoutedSharedMoEWeights",
    "PreparedW8A16TiledFusedMoEWeights", "PreparedW8A8TiledFusedMoEWeights",
    "PreparedW8A16TiledRoutedSharedMoEWeights", "PreparedW8A8TiledRoutedSharedMoEWeights",
    "_HAS_BF16_TILED_FUSED_MOE", "_HAS_W8A8_TILED_FUSED_MOE", "available_fused_moe_bf16_tiled_backends",
    "calibrate_moe_planner_quick", "enable_moe_planner_quick", "fused_moe_bf16_tiled",
    "fused_moe_bf16_tiled_with_shared", "fused_moe_bf16_tiled_scheduled", "fused_moe_bf16_tiled_async",
    "fused_moe_bf16_tiled_async_plan", "fused_moe_bf16_tiled_planned_staged", "fused_moe_bf16_tiled_vllm_staged",
    "fused_moe_tiled", "fused_moe_w8a16_tiled", "fused_moe_w8a16_tiled_async_plan", "fused_moe_w8a8_tiled",
    "fused_moe_w8a8_tiled_async_plan", "fused_moe_w8a16_tiled_with_shared", "fused_moe_w8a8_tiled_with_shared",
    "shared_mlp_bf16_tiled", "fused_moe_naive", "get_default_moe_planner_runtime", "bf16_tiled_fused_moe",
    "bf16_tiled_fused_moe_scheduled", "bf16_tiled_fused_moe_async", "bf16_tiled_fused_moe_async_plan",
    "bf16_tiled_fused_moe_planned_staged", "bf16_tiled_fused_moe_vllm_staged", "naive_fused_moe",
    "prepare_fused_moe_bf16_tiled_weights", "prepare_fused_moe_w8a16_tiled_weights",
    "prepare_fused_moe_w8a16_tiled_quantized_weights", "prepare_fused_moe_w8a8_tiled_weights",
    "prepare_fused_moe_w8a8_tiled_quantized_weights", "prepare_routed_shared_moe_bf16_tiled_weights",
    "prepare_routed_shared_moe_w8a16_tiled_quantized_weights",
    "prepare_routed_shared_moe_w8a8_tiled_quantized_weights", "prepare_shared_mlp_bf16_tiled_weights",
    "prepare_bf16_tiled_fused_moe_weights", "set_default_moe_planner_runtime", "upgrade_legacy_async_plan",
}
# the torch-op reference implementation is not part of the GPU operator surface
NOT_MIRRORED = {"fused_moe_naive", "naive_fused_moe"}

REFERENCE_I8GEMM_ALL = {"PreparedI8GEMMWeight", "_supports_i8gemm", "dynamic_scaled_mm", "dynamic_scaled_mm_pair",
                        "mm", "prepare"}


def _declared_symbols() -> set[str]:
    text = (REPO / "include" / "fcmoe.h").read_text()
    return set(re.findall(r"\b(fcmoe_[a-z0-9_]+)\s*\(", text))


def test_cabi_library_exports_every_declared_symbol():
    from fused_cpp_amd import cabi

    lib = ctypes.CDLL(str(cabi.LIB_PATH))
    declared = _declared_symbols()
    assert len(declared) >= 19
    missing = [name for name in sorted(declared) if not hasattr(lib, name)]
    assert not missing, f"libfcmoe.so lacks {missing}"
    assert set(cabi.SIGNATURES) == declared  # the ctypes binding covers the whole header


def test_cabi_host_only_calls():
    from fused_cpp_amd import cabi

    L = cabi.lib()
    assert L.fcmoe_abi_version() == 1
    assert L.fcmoe_packed_expert_bytes(1, 4096, 7168, 2) == 4096 * 7168
    assert L.fcmoe_packed_expert_bytes(2, 22, 13, 2) == 2 * 16 * 64
    assert L.fcmoe_packed_expert_bytes(3, 16, 16, 1) == -1
    assert L.fcmoe_route_workspace_bytes(64, 8, 257, 256) > 0
    args = cabi.MoeArgs()
    args.tokens, args.hidden, args.inter, args.top_k, args.experts, args.valid_experts = 64, 7168, 2048, 8, 257, 257
    args.shared_expert_id = 256
    assert L.fcmoe_w8a8_workspace_bytes(ctypes.byref(args)) > 64 * 9 * 7168 * 4
    # argument validation happens before any device work
    args.activation = cabi.FCMOE_ACT_SILU
    assert L.fcmoe_w8a8_forward(ctypes.byref(args), None) == -1
    assert b"limit 10" in L.fcmoe_last_error()
    args.experts = 2000
    assert L.fcmoe_bf16_forward(ctypes.byref(args), None) == -1
    assert b"experts" in L.fcmoe_last_error()


def test_extension_module_loads():
    from fused_cpp_amd import _native

    assert _native.moe_C is not None, _native.NATIVE_ERROR
    for name in ("fused_moe_w8a8_forward", "fused_moe_bf16_forward", "fused_moe_w8a8_prepare_weights",
                 "fused_moe_bf16_prepare_weights", "i8gemm_prepare", "i8gemm_dynamic_scaled_mm"):
        assert hasattr(_native.moe_C, name)


def test_python_surface_mirrors_reference():
    import fused_cpp_amd.i8gemm as i8
    import fused_cpp_amd.moe as moe

    assert REFERENCE_MOE_ALL - NOT_MIRRORED <= set(moe.__all__)
    assert REFERENCE_I8GEMM_ALL <= set(i8.__all__)
    w = moe.PreparedW8A8TiledFusedMoEWeights(w13=(torch.empty(1), 16, 16, torch.empty(1)),
                                             w2=(torch.empty(1), 16, 16, torch.empty(1)))
    assert w.fused_silu and w.backend_n_tile == 16


def test_plan_v2_schema_shims():
    from fused_cpp_amd.moe import AsyncMoEPlanV2, upgrade_legacy_async_plan

    raw = upgrade_legacy_async_plan({"num_threads": 4, "thread_cpu_ids": [0, 1, 2, 3], "task_expert_ids": [0, 1],
                                     "task_core_begins": [0, 2], "task_threads": [2, 2],
                                     "task_dep_offsets": [0, 0, 0], "task_deps": []})
    plan = AsyncMoEPlanV2.from_dict(raw)
    assert plan.plan_version == 2 and plan.native_execution_mode == 0 and plan.native_early_merge == -1
    with pytest.raises(ValueError, match="plan_version"):
        AsyncMoEPlanV2.from_dict({**raw, "plan_version": 1})
    with pytest.raises(ValueError, match="missing"):
        AsyncMoEPlanV2.from_dict({"plan_version": 2})


def test_planner_runtime_shims():
    from fused_cpp_amd.moe import (MoePlannerRuntime, enable_moe_planner_quick, get_default_moe_planner_runtime,
                                   set_default_moe_planner_runtime)

    rt = enable_moe_planner_quick(hidden_size=7168, intermediate_size=2048, global_experts=256, local_experts=256,
                                  shared_experts=1)
    assert get_default_moe_planner_runtime() is rt
    assert rt.plan_for_dispatch(None, None) is None
    assert set_default_moe_planner_runtime(None) is rt
    with pytest.raises(TypeError):
        set_default_moe_planner_runtime(object())
    with pytest.raises(ValueError):
        MoePlannerRuntime(None, hidden_size=1, intermediate_size=1, global_experts=1, local_experts=1,
                          shared_experts=2)


@pytest.fixture
def fake_backend(monkeypatch):
    """Make the wrappers believe a device exists and route native calls to a recorder."""
    from fused_cpp_amd.moe import bf16_tiled as mod

    calls = {}
    monkeypatch.setattr(mod, "_require_backend", lambda: None)
    monkeypatch.setattr(mod, "_check_device_tensor", lambda t, name: None)

    class FakeC:
        def fused_moe_w8a8_forward(self, *args):
            calls["w8a8"] = args
            return args[0]

        def fused_moe_bf16_forward(self, *args):
            calls["bf16"] = args
            return args[0]

    monkeypatch.setattr(mod._native, "moe_C", FakeC())
    return mod, calls


def test_w8a8_routed_shared_wrapper_passes_shared_slot(fake_backend):
    mod, calls = fake_backend
    packed = mod.PreparedW8A8TiledFusedMoEWeights(w13=(torch.empty((3, 8)), 16, 32, torch.ones(3, 32)),
                                                  w2=(torch.empty((3, 8)), 16, 16, torch.ones(3, 16)))
    weights = mod.PreparedW8A8TiledRoutedSharedMoEWeights(packed=packed, routed_experts=2, shared_expert_id=2)
    x = torch.zeros((2, 16), dtype=torch.bfloat16)
    ids = torch.tensor([[0, 1], [1, 0]], dtype=torch.int64)
    w = torch.tensor([[0.7, 0.3], [0.4, 0.6]], dtype=torch.float32)
    mod.fused_moe_w8a8_tiled_with_shared(x, weights, w, ids, num_threads=4, routed_scaling_factor=2.5,
                                         swiglu_limit=10.0)
    args = calls["w8a8"]
    assert args[11] == 2 and args[12] == 2.5 and args[13] == 2  # shared id, scale, routed ids < 2
    assert torch.equal(args[10], ids)


def test_w8a8_wrappers_reject_reference_error_cases(fake_backend):
    mod, _ = fake_backend
    w = mod.PreparedW8A8TiledFusedMoEWeights(w13=(torch.empty((1, 8)), 16, 16, torch.ones(1, 16)),
                                             w2=(torch.empty((1, 8)), 8, 16, torch.ones(1, 16)))
    x = torch.zeros((1, 16), dtype=torch.bfloat16)
    ids = torch.zeros((1, 1), dtype=torch.int64)
    with pytest.raises(ValueError, match="swiglu_limit=10.0"):
        mod.fused_moe_w8a8_tiled_async_plan(x, w, torch.ones((1, 1)), ids, {"plan_version": 2}, swiglu_limit=0.0)
    with pytest.raises(TypeError):
        mod.fused_moe_w8a8_tiled(x, "not weights", torch.ones((1, 1)), ids)
    with pytest.raises(RuntimeError, match="global_num_experts"):
        mod.fused_moe_w8a8_tiled(x, w, torch.ones((1, 1)), ids, global_num_experts=4)
    with pytest.raises(TypeError, match="integer"):
        mod.fused_moe_w8a8_tiled(x, w, torch.ones((1, 1)), torch.zeros((1, 1)))


def test_bf16_wrapper_activation_and_limit_rules(fake_backend):
    mod, calls = fake_backend
    w = mod.PreparedBF16TiledFusedMoEWeights(w13=(torch.empty((1, 8)), 16, 16), w2=(torch.empty((1, 8)), 8, 16),
                                             fused_silu=True)
    x = torch.zeros((1, 16), dtype=torch.bfloat16)
    ids = torch.zeros((1, 1), dtype=torch.int32)
    mod.fused_moe_bf16_tiled(x, w, torch.ones((1, 1)), ids, swiglu_limit=10.0)
    assert calls["bf16"][11] == "silu_clamp10"
    mod.fused_moe_bf16_tiled(x, w, torch.ones((1, 1)), ids, swiglu_limit=0.0)
    assert calls["bf16"][11] == "silu"
    with pytest.raises(ValueError, match="swiglu_limit=10.0"):
        mod.fused_moe_bf16_tiled(x, w, torch.ones((1, 1)), ids, swiglu_limit=7.0)
    with pytest.raises(ValueError, match="Unsupported MoE activation"):
        mod.fused_moe_bf16_tiled(x, w, torch.ones((1, 1)), ids, activation="relu")
    with pytest.raises(ValueError, match="skip_weighted"):
        mod.fused_moe_bf16_tiled(x, w, torch.ones((1, 2)), torch.zeros((1, 2), dtype=torch.int32),
                                 skip_weighted=True)
    nf = mod.PreparedBF16TiledFusedMoEWeights(w13=(torch.empty((1, 8)), 16, 16), w2=(torch.empty((1, 8)), 8, 16))
    with pytest.raises(ValueError, match="fuse_silu"):
        mod.fused_moe_bf16_tiled(x, nf, torch.ones((1, 1)), ids, swiglu_limit=10.0)
    with pytest.raises(ValueError, match="out must have shape"):
        mod.fused_moe_bf16_tiled(x, w, torch.ones((1, 1)), ids, out=torch.empty((2, 16), dtype=torch.bfloat16))


def test_fused_moe_tiled_dispatches_on_weight_type(fake_backend, monkeypatch):
    mod, _ = fake_backend
    w8 = mod.PreparedW8A8TiledFusedMoEWeights(w13=(torch.empty(1), 16, 16, torch.empty(1)),
                                              w2=(torch.empty(1), 16, 16, torch.empty(1)))
    expected = torch.zeros((1, 16), dtype=torch.bfloat16)
    monkeypatch.setattr(mod, "fused_moe_w8a8_tiled", lambda *a, **k: expected)
    assert mod.fused_moe_tiled(expected, w8, torch.ones((1, 1)), torch.zeros((1, 1), dtype=torch.int64),
                               swiglu_limit=10.0) is expected
    with pytest.raises(ValueError, match="bias"):
        mod.fused_moe_tiled(expected, w8, torch.ones((1, 1)), torch.zeros((1, 1), dtype=torch.int64),
                            w13_bias=torch.zeros(1))
    with pytest.raises(TypeError):
        mod.fused_moe_tiled(expected, object(), torch.ones((1, 1)), torch.zeros((1, 1), dtype=torch.int64))


def test_w8a16_entry_points_fail_loudly_without_a_gpu():
    """No CPU fallback: on a host without a ROCm device every W8A16 entry raises."""
    from fused_cpp_amd import moe

    for fn, args in ((moe.fused_moe_w8a16_tiled, (None, None, None, None)),
                     (moe.fused_moe_w8a16_tiled_with_shared, (None, None, None, None)),
                     (moe.prepare_fused_moe_w8a16_tiled_weights, (None, None)),
                     (moe.prepare_fused_moe_w8a16_tiled_quantized_weights, (None, None, None, None))):
        with pytest.raises(RuntimeError, match="ROCm device"):
            fn(*args)


def test_deepseek_v4_w8a8_surface_matches_reference_names():
    """src/fused_cpp/deepseek_v4_w8a8.py __all__; entry points fail loudly without a GPU."""
    from fused_cpp_amd import deepseek_v4_w8a8 as ds

    assert set(ds.__all__) == {
        "PreparedDeepSeekV4W8A8LinearWeight", "_HAS_DEEPSEEK_V4_W8A8", "deepseek_v4_w8a8_linear",
        "deepseek_v4_w8a8_linear_pair", "deepseek_v4_wo_b_w8a8", "prepare_deepseek_v4_w8a8_linear_quantized_weight",
        "prepare_deepseek_v4_w8a8_linear_weight"}
    if not ds._HAS_DEEPSEEK_V4_W8A8:
        with pytest.raises(RuntimeError):
            ds.prepare_deepseek_v4_w8a8_linear_weight(torch.zeros((4, 8), dtype=torch.bfloat16))


def test_bench_torch_eager_baseline_matches_oracle():
    """bench.py's CPU baseline (the reference test's eager formula, grouped per
    expert) computes the same layer as the oracle: within a few bf16 ulps (it
    rounds ties to even and uses torch.exp where the reference kernel rounds
    half away and uses its FEXPA exp)."""
    import numpy as np
    import torch

    import bench
    import oracle
    from tests import helpers as H

    cfg = dict(kind="w8a8", T=40, H=256, I=128, E=6, k=3, shared=True, scale=2.5, skew=None)
    x, ids, w, q13, s13, q2, s2 = H.w8a8_case(3, 40, 256, 128, 7, 3)
    ids = ids % 6
    experts = np.arange(7)
    routes, _ = bench._expert_routes(cfg, ids, experts)
    xb = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    got = bench.torch_eager_expert_layer(xb, ids, w, cfg, experts, (q13, s13, q2, s2), routes)
    ref = H.bits_to_f32(oracle.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=6, routed_scale=2.5))
    got = got.to(torch.bfloat16).float().numpy()
    assert np.abs(got - ref).max() <= 2e-2 * max(1.0, np.abs(ref).max())
    # a uniform expert sample and its complement add up to the whole layer
    a = bench.torch_eager_expert_layer(xb, ids, w, cfg, experts[:3], (q13[:3], s13[:3], q2[:3], s2[:3]), routes[:3])
    b = bench.torch_eager_expert_layer(xb, ids, w, cfg, experts[3:], (q13[3:], s13[3:], q2[3:], s2[3:]), routes[3:])
    full = bench.torch_eager_expert_layer(xb, ids, w, cfg, experts, (q13, s13, q2, s2), routes)
    np.testing.assert_allclose((a + b).numpy(), full.numpy(), rtol=1e-5, atol=1e-5)


def test_noalloc_rejects_calls_beyond_its_scratch():
    """The fixed-scratch W8A8 entry point refuses a call whose workspace would
    exceed the array, before touching the device (so this runs without a GPU)."""
    import ctypes

    from fused_cpp_amd import cabi

    L = cabi.lib()
    a = cabi.MoeArgs()
    a.tokens, a.hidden, a.inter = 4096, 7168, 2048
    a.top_k, a.experts, a.valid_experts, a.shared_expert_id = 8, 257, 257, 256
    a.routed_scaling = 2.5
    a.activation = cabi.FCMOE_ACT_SILU_CLAMP10
    assert L.fcmoe_w8a8_workspace_bytes(ctypes.byref(a)) > cabi.FCMOE_NOALLOC_SCRATCH_BYTES
    rc = L.fcmoe_w8a8_forward_noalloc(ctypes.byref(a), None)
    assert rc == -2  # FCMOE_ESPACE
    assert "scratch" in L.fcmoe_last_error().decode()
    a.tokens = 64  # C2's decode batch fits the array
    assert L.fcmoe_w8a8_workspace_bytes(ctypes.byref(a)) <= cabi.FCMOE_NOALLOC_SCRATCH_BYTES


def test_w8a8_prefill_plan_choice(monkeypatch):
    """The library's prefill launch-plan rule on the route scan's per-class
    tile counts (host side; the device evaluates the same inline function):
    mixed with >= 32 tiles of 16 rows and >= 16 of 256 rows, otherwise the
    classic plan, partitioned when the 256-row class is a minority of the
    weighted work (2.5 x a 128/192-row tile, 20 x a 16-row tile), on
    [32, 128] CUs rounded down to the 8 XCDs."""
    from fused_cpp_amd import cabi

    monkeypatch.delenv("FCMOE_PREFILL_MIXED_MIN_TILES", raising=False)
    monkeypatch.delenv("FCMOE_PREFILL_PART", raising=False)
    assert cabi.w8a8_prefill_plan([149, 20, 15, 140]) == ("mixed", 0)  # C3-like
    assert cabi.w8a8_prefill_plan([31, 0, 0, 140])[0] != "mixed"
    assert cabi.w8a8_prefill_plan([149, 20, 15, 15])[0] != "mixed"
    # C4: 364 experts of 129-192 rows, 52 tiles of 256 rows: 256 * 1040 / 3952 = 67 -> 64
    assert cabi.w8a8_prefill_plan([0, 0, 364, 52]) == ("partitioned", 64)
    assert cabi.w8a8_prefill_plan([0, 256, 0, 8]) == ("partitioned", 32)  # clamped up to 32
    assert cabi.w8a8_prefill_plan([0, 0, 0, 288]) == ("classic", 0)  # the 256-row class dominates
    assert cabi.w8a8_prefill_plan([5, 10, 0, 0]) == ("classic", 0)  # no 256-row tiles
    monkeypatch.setenv("FCMOE_PREFILL_PART", "0")
    assert cabi.w8a8_prefill_plan([0, 0, 364, 52]) == ("classic", 0)
    monkeypatch.setenv("FCMOE_PREFILL_MIXED_MIN_TILES", "0")
    assert cabi.w8a8_prefill_plan([0, 0, 364, 52]) == ("mixed", 0)
    with pytest.raises(RuntimeError):
        cabi.check(cabi.lib().fcmoe_w8a8_prefill_plan(None, None), "plan")


def test_bf16_half_ulp_bounds_bf16_rounding():
    """The allowance the BF16 tolerance checks add for the output's own
    rounding: it bounds |bf16(x) - x| (round to nearest even, the oracle's
    converter) and is reached, i.e. it is exactly half a bf16 ulp."""
    import numpy as np

    import oracle
    from tests import helpers as H

    rng = np.random.default_rng(3)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-6, 6, 200000))).astype(np.float32)
    r = H.bits_to_f32(oracle.f32_to_bf16_bits(x)).astype(np.float64)
    err = np.abs(r - x.astype(np.float64))
    half = H.bf16_half_ulp(x)
    assert (err <= half).all()
    assert (err / half).max() > 0.999
    assert H.bf16_half_ulp(np.array([1.0, 10.0, 0.75]))[1] == 2.0 ** -5


def test_i8gemm_pair_workspace_covers_both_gemms():
    """The pair's two GEMMs can split K differently (the split count depends
    on N): its workspace must hold the larger partial-sum area, whichever GEMM
    needs it (a pair sized for max(N) alone once left the second GEMM's partial
    sums past the end of the workspace)."""
    from fused_cpp_amd import cabi

    L = cabi.lib()
    for m in (1, 16, 33, 64, 65, 300):
        for k in (64, 1536, 7168, 16384):
            for n1, n2 in ((24576, 8192), (8192, 24576), (7168, 7168), (100, 65536), (32768, 512)):
                pair = L.fcmoe_i8gemm_pair_workspace_bytes(m, k, n1, n2)
                assert pair >= L.fcmoe_i8gemm_workspace_bytes(m, k, n1), (m, k, n1, n2)
                assert pair >= L.fcmoe_i8gemm_workspace_bytes(m, k, n2), (m, k, n1, n2)
