"""GPU tests of the public operator surface (fused_cpp_amd.moe / .i8gemm),
mirroring the reference's operator tests (tests/test_fused_moe_bf16_tiled.py,
tests/test_shared_mlp_bf16_tiled.py, tests/test_moe_w8a8.py,
tests/test_i8gemm.py, tests/test_deepseek_v4_w8a8.py).

Bars: W8A8 and i8gemm are bit-exact against the oracle. BF16 is compared with
the fp32 reference (oracle.bf16_moe_reference, naive.py semantics) within
max|out - ref| <= 2e-2 * max(1, max|ref|) and cosine >= 0.9999 (the north-star
bound, relative to the output scale), plus the reference tests' own
tolerances where they apply (7e-2, clamp 0.25/0.08). Routed+shared and shared
MLP invariants are exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _bf16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(H.bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _close(out: torch.Tensor, ref: np.ndarray, tol: float = 2e-2, cos_min: float = 0.9999) -> None:
    o = out.float().cpu().numpy().astype(np.float64)
    r = ref.astype(np.float64)
    scale = max(1.0, float(np.abs(r).max()))
    err = float(np.abs(o - r).max())
    cos = float((o * r).sum() / np.sqrt((o * o).sum() * (r * r).sum() + 1e-300))
    assert err <= tol * scale, f"max-abs {err:.4e} > {tol} * {scale:.3f}"
    assert cos >= cos_min, f"cosine {cos:.7f} < {cos_min}"


# ------------------------------------------------------------------- W8A8 --

def _w8a8_weights(case, shared: bool, dev):
    from fused_cpp_amd import moe

    x, ids, w, q13, s13, q2, s2 = case
    T = lambda a: torch.from_numpy(a)  # noqa: E731  (host tensors: prepare moves them)
    if shared:
        return moe.prepare_routed_shared_moe_w8a8_tiled_quantized_weights(
            T(q13[:-1]), T(s13[:-1]), T(q2[:-1]), T(s2[:-1]), T(q13[-1]), T(s13[-1]), T(q2[-1]), T(s2[-1]))
    return moe.prepare_fused_moe_w8a8_tiled_quantized_weights(T(q13), T(s13), T(q2), T(s2))


@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_w8a8_with_shared_public_api_bit_exact(gpu, oracle_lib, ids_dtype):
    from fused_cpp_amd import moe

    case = H.w8a8_case(5, 48, 512, 256, 13, 4)
    x, ids, w, q13, s13, q2, s2 = case
    ids = np.minimum(ids, 11)
    prepared = _w8a8_weights(case, True, gpu)
    xt = torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.bfloat16)
    out = torch.empty_like(xt)
    got = moe.fused_moe_w8a8_tiled_with_shared(xt, prepared, torch.from_numpy(w).to(gpu),
                                               torch.from_numpy(ids).to(gpu).to(ids_dtype),
                                               routed_scaling_factor=2.5, out=out)
    assert got is out
    ref = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2, shared_id=12, routed_scale=2.5)
    np.testing.assert_array_equal(_bits(got), ref)
    again = moe.fused_moe_w8a8_tiled_with_shared(xt, prepared, torch.from_numpy(w).to(gpu),
                                                 torch.from_numpy(ids).to(gpu), routed_scaling_factor=2.5)
    np.testing.assert_array_equal(_bits(again), ref)  # repeat bitwise (tests/test_moe_w8a8.py:226)


def test_w8a8_tiled_and_plan_entry_points_bit_exact(gpu, oracle_lib):
    from fused_cpp_amd import moe

    case = H.w8a8_case(23, 48, 64, 64, 2, 1, int_range=12)
    x, ids, w, q13, s13, q2, s2 = case
    prepared = _w8a8_weights(case, False, gpu)
    xt = torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.bfloat16)
    wt, it = torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu)
    ref = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2)
    plan = moe.upgrade_legacy_async_plan({"num_threads": 2, "thread_cpu_ids": [0, 1], "task_expert_ids": [0, 1],
                                          "task_core_begins": [0, 1], "task_threads": [1, 1],
                                          "task_dep_offsets": [0, 0, 0], "task_deps": []})
    for got in (moe.fused_moe_w8a8_tiled(xt, prepared, wt, it),
                moe.fused_moe_w8a8_tiled_async_plan(xt, prepared, wt, it, plan),
                moe.fused_moe_tiled(xt, prepared, wt, it, swiglu_limit=10.0)):
        np.testing.assert_array_equal(_bits(got), ref)


def test_w8a8_prepare_from_bf16_matches_oracle_quantisation(gpu, oracle_lib):
    from fused_cpp_amd import moe

    rng = np.random.default_rng(8)
    E, Hd, F, T, k = 3, 128, 64, 16, 2
    w13 = H.bf16_bits(rng.standard_normal((E, 2 * F, Hd)).astype(np.float32) * 0.02)
    w2 = H.bf16_bits(rng.standard_normal((E, Hd, F)).astype(np.float32) * 0.02)
    w13[0, 5] = 0  # an all-zero channel: scale 1
    prepared = moe.prepare_fused_moe_w8a8_tiled_weights(torch.from_numpy(w13.view(np.int16)).view(torch.bfloat16),
                                                        torch.from_numpy(w2.view(np.int16)).view(torch.bfloat16))
    q13, s13 = oracle_lib.quant_weight_rows(w13)
    q2, s2 = oracle_lib.quant_weight_rows(w2)
    np.testing.assert_array_equal(prepared.w13[3].cpu().numpy(), s13)
    np.testing.assert_array_equal(prepared.w2[3].cpu().numpy(), s2)
    x = H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32))
    ids, w = H.softmax_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    got = moe.fused_moe_w8a8_tiled(torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.bfloat16), prepared,
                                   torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu))
    np.testing.assert_array_equal(_bits(got), oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2))


def test_w8a8_invalid_ids_raise(gpu):
    from fused_cpp_amd import moe

    case = H.w8a8_case(2, 8, 64, 64, 3, 2)
    x, ids, w, *_ = case
    prepared = _w8a8_weights(case, True, gpu)
    xt = torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.bfloat16)
    bad = torch.from_numpy(ids).to(gpu).clone()
    bad[0, 0] = 2  # the shared expert id is not a valid routed id
    with pytest.raises(ValueError, match="routed topk_ids"):
        moe.fused_moe_w8a8_tiled_with_shared(xt, prepared, torch.from_numpy(w).to(gpu), bad)
    plain = _w8a8_weights(case, False, gpu)
    bad[0, 0] = 7
    with pytest.raises(RuntimeError, match="out of range"):
        moe.fused_moe_w8a8_tiled(xt, plain, torch.from_numpy(w).to(gpu), bad)


@pytest.mark.parametrize("T", [1, 40, 600])
def test_w8a8_id_check_alternating_calls(gpu, monkeypatch, T):
    """The id check (a pinned host count the host polls while the forward
    runs) across calls: valid, invalid, valid again, behind queued GPU work;
    one token (decode head), the small route and the 3-kernel route (1200
    routes). Results with the check equal those without it, bit for bit."""
    from fused_cpp_amd import moe

    case = H.w8a8_case(11 + T, T, 256, 128, 5, 2)
    x, ids, w, *_ = case
    plain = _w8a8_weights(case, False, gpu)
    xt = torch.from_numpy(x.view(np.int16)).to(gpu).view(torch.bfloat16)
    wt = torch.from_numpy(w).to(gpu)
    good = torch.from_numpy(ids).to(gpu)
    bad = good.clone()
    bad[T - 1, 1] = 5
    monkeypatch.setenv("FUSED_CPP_AMD_VALIDATE_IDS", "0")
    ref = _bits(moe.fused_moe_w8a8_tiled(xt, plain, wt, good))
    monkeypatch.setenv("FUSED_CPP_AMD_VALIDATE_IDS", "1")
    big = torch.randn(4096, 4096, device=gpu)
    for rep in range(3):
        _ = big @ big  # queued ahead of the forward: the host waits for the route launch, not the stream
        assert np.array_equal(_bits(moe.fused_moe_w8a8_tiled(xt, plain, wt, good)), ref), rep
        with pytest.raises(RuntimeError, match="1 id\\(s\\) outside"):
            moe.fused_moe_w8a8_tiled(xt, plain, wt, bad)
    torch.cuda.synchronize()


def test_w8a8_empty_input(gpu):
    from fused_cpp_amd import moe

    case = H.w8a8_case(2, 4, 64, 64, 3, 2)
    prepared = _w8a8_weights(case, False, gpu)
    x = torch.empty((0, 64), dtype=torch.bfloat16, device=gpu)
    out = moe.fused_moe_w8a8_tiled(x, prepared, torch.empty((0, 2), device=gpu),
                                   torch.empty((0, 2), dtype=torch.int64, device=gpu))
    assert out.shape == (0, 64)


def test_w8a8_full_size_prefill_sampled_tokens_bit_exact(gpu, oracle_lib):
    """T=4096 at DSv3 H/F with Zipf-skewed routing over 64 experts + shared:
    the whole layer on the GPU, a sample of tokens recomputed by the oracle
    (its per-token arithmetic is independent of the other tokens)."""
    case = H.w8a8_case(77, 4096, 7168, 2048, 65, 8, skew=1.2)
    x, ids, w, q13, s13, q2, s2 = case
    ids = np.minimum(ids, 63)
    out = H.gpu_w8a8_forward(x, ids, w, q13, s13, q2, s2, gpu, shared_id=64, scale=2.5)
    sample = np.random.default_rng(0).choice(4096, 48, replace=False)
    ref = oracle_lib.w8a8_forward(x[sample], ids[sample], w[sample], q13, s13, q2, s2, shared_id=64,
                                  routed_scale=2.5)
    np.testing.assert_array_equal(out[sample], ref)


# ------------------------------------------------------------------- BF16 --

def _bf16_case(seed, T, Hd, F, E, k, bias=True, w_std=1.0):
    """The reference's _case (tests/test_fused_moe_bf16_tiled.py:57-82) shape family."""
    rng = np.random.default_rng(seed)
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bits_to_f32(H.bf16_bits(rng.standard_normal((E, 2 * F, Hd)).astype(np.float32) * w_std))
    w2 = H.bits_to_f32(H.bf16_bits(rng.standard_normal((E, Hd, F)).astype(np.float32) * w_std))
    b13 = (rng.standard_normal((E, 2 * F)) * 0.1).astype(np.float32) if bias else None
    b2 = (rng.standard_normal((E, Hd)) * 0.1).astype(np.float32) if bias else None
    ids = np.array([[(i + j) % E for j in range(k)] for i in range(T)], np.int32)
    lw = rng.standard_normal((T, k)).astype(np.float32)
    w = np.exp(lw) / np.exp(lw).sum(1, keepdims=True)
    return x, w13, w2, b13, b2, ids, w.astype(np.float32)


@pytest.mark.parametrize("activation", ["silu", "swigluoai", "gelu"])
def test_bf16_matches_naive_reference(gpu, oracle_lib, activation):
    """tests/test_fused_moe_bf16_tiled.py:1692-1728: vs fused_moe_naive at atol=rtol=7e-2."""
    from fused_cpp_amd import moe

    x, w13, w2, b13, b2, ids, w = _bf16_case(123, 37, 13, 11, 4, 2)
    packed = moe.prepare_fused_moe_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu))
    out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu),
                                   w13_bias=torch.from_numpy(b13).to(gpu), w2_bias=torch.from_numpy(b2).to(gpu),
                                   activation=activation)
    ref = oracle_lib.bf16_moe_reference(x, w13, w2, w, ids, w13_bias=b13, w2_bias=b2, activation=activation)
    refb = torch.from_numpy(ref).to(torch.bfloat16).float()
    torch.testing.assert_close(out.float().cpu(), refb, atol=7e-2, rtol=7e-2)


def test_bf16_clamped_swiglu_matches_reference(gpu, oracle_lib):
    """tests/test_fused_moe_bf16_tiled.py:267-355: limit 10 vs fp32, 0 == unclamped."""
    from fused_cpp_amd import moe

    rng = np.random.default_rng(20260818)
    counts = list(range(1, 13))
    E, T, Hd, F = len(counts), sum(counts), 64, 32
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bits_to_f32(H.bf16_bits(rng.standard_normal((E, 2 * F, Hd)).astype(np.float32)))
    w2 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E, Hd, F)) * 0.02).astype(np.float32)))
    ids = np.concatenate([np.full(c, e) for e, c in enumerate(counts)]).reshape(-1, 1).astype(np.int32)
    w = np.ones((T, 1), np.float32)
    packed = moe.prepare_fused_moe_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu), fuse_silu=True)
    args = (_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu))
    unclamped = moe.fused_moe_bf16_tiled(*args)
    zero = moe.fused_moe_bf16_tiled(*args, swiglu_limit=0.0)
    clamped = moe.fused_moe_bf16_tiled(*args, swiglu_limit=10.0)
    assert torch.equal(zero, unclamped)
    ref = oracle_lib.bf16_moe_reference(x, w13, w2, w, ids, activation="silu_clamp10", round_intermediate=True)
    torch.testing.assert_close(clamped.float().cpu(), torch.from_numpy(ref).to(torch.bfloat16).float(), atol=0.25,
                               rtol=0.08)
    assert float((clamped.float() - unclamped.float()).abs().max()) > 0.5


def test_bf16_skip_weighted_and_global_experts(gpu, oracle_lib):
    from fused_cpp_amd import moe

    x, w13, w2, b13, b2, ids, _ = _bf16_case(7, 37, 13, 11, 4, 1)
    w = np.ones((37, 1), np.float32)
    packed = moe.prepare_fused_moe_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu))
    out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu),
                                   w13_bias=torch.from_numpy(b13).to(gpu), w2_bias=torch.from_numpy(b2).to(gpu),
                                   skip_weighted=True, global_num_experts=4)
    ref = oracle_lib.bf16_moe_reference(x, w13, w2, w, ids, w13_bias=b13, w2_bias=b2, skip_weighted=True)
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref).to(torch.bfloat16).float(), atol=7e-2,
                               rtol=7e-2)
    with pytest.raises(RuntimeError, match="out of range"):
        moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu),
                                 global_num_experts=2)


@pytest.mark.parametrize("T,Hd,F,E,k", [(32, 1024, 512, 8, 2), (5, 256, 128, 8, 6), (40, 512, 96, 6, 4)])
def test_bf16_plumbing_config_within_north_star_tolerance(gpu, oracle_lib, T, Hd, F, E, k):
    """BASELINE configs[0] (C0) and tree-merge top-k variants vs the fp32 reference."""
    from fused_cpp_amd import moe

    rng = np.random.default_rng(T * Hd + k)
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E, 2 * F, Hd)) * 0.02).astype(np.float32)))
    w2 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E, Hd, F)) * 0.02).astype(np.float32)))
    ids, w = H.softmax_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    packed = moe.prepare_fused_moe_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu), fuse_silu=True)
    out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu))
    _close(out, oracle_lib.bf16_moe_reference(x, w13, w2, w, ids))


def test_bf16_more_routes_than_grid_y_limit(gpu, oracle_lib):
    """65,600 routes (T=8200, top-8): row-indexed passes (activation, combine)
    cover every row although a launch's grid.y stops at 65,535."""
    from fused_cpp_amd import moe

    x, w13, w2, b13, b2, ids, w = _bf16_case(8200, 8200, 64, 32, 8, 8, w_std=0.1)
    packed = moe.prepare_fused_moe_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu))
    out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu),
                                   w13_bias=torch.from_numpy(b13).to(gpu), w2_bias=torch.from_numpy(b2).to(gpu),
                                   activation="swigluoai")
    ref = oracle_lib.bf16_moe_reference(x, w13, w2, w, ids, w13_bias=b13, w2_bias=b2, activation="swigluoai")
    refb = torch.from_numpy(ref).to(torch.bfloat16).float()
    torch.testing.assert_close(out.float().cpu(), refb, atol=7e-2, rtol=7e-2)
    # the last rows are as close as the first (no row left unwritten)
    torch.testing.assert_close(out[-64:].float().cpu(), refb[-64:], atol=7e-2, rtol=7e-2)


def test_w8a8_more_tokens_than_grid_y_limit(gpu, oracle_lib):
    """70,000 tokens: the combine strides over tokens past grid.y's 65,535."""
    case = H.w8a8_case(70000, 70000, 64, 32, 4, 1)
    x, ids, w, q13, s13, q2, s2 = case
    out = H.gpu_w8a8_forward(x, ids, w, q13, s13, q2, s2, gpu)
    ref = oracle_lib.w8a8_forward(x, ids, w, q13, s13, q2, s2)
    np.testing.assert_array_equal(out, ref)


def test_bf16_dsv3_shape_routed_shared_within_tolerance(gpu, oracle_lib):
    """C1 shape (H=7168, I=2048, top-8 + shared, x2.5) with 16 routed experts."""
    from fused_cpp_amd import moe

    rng = np.random.default_rng(11)
    T, Hd, F, E, k = 32, 7168, 2048, 16, 8
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E + 1, 2 * F, Hd)) * 0.02).astype(np.float32)))
    w2 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E + 1, Hd, F)) * 0.02).astype(np.float32)))
    ids, w = H.softmax_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    prepared = moe.prepare_routed_shared_moe_bf16_tiled_weights(_bf16(w13[:E], gpu), _bf16(w2[:E], gpu),
                                                                _bf16(w13[E], gpu), _bf16(w2[E], gpu))
    out = moe.fused_moe_bf16_tiled_with_shared(_bf16(x, gpu), prepared, torch.from_numpy(w).to(gpu),
                                               torch.from_numpy(ids).to(gpu), routed_scaling_factor=2.5)
    ids_c = np.concatenate([ids, np.full((T, 1), E)], 1)
    w_c = np.concatenate([w * np.float32(2.5), np.ones((T, 1), np.float32)], 1)
    _close(out, oracle_lib.bf16_moe_reference(x, w13, w2, w_c, ids_c))


def test_routed_shared_equals_explicit_combined_route(gpu):
    """tests/test_shared_mlp_bf16_tiled.py:148-231: exact."""
    from fused_cpp_amd import moe

    x, w13, w2, _, _, ids, w = _bf16_case(31, 19, 192, 96, 5, 2, bias=False, w_std=0.05)
    prepared = moe.prepare_routed_shared_moe_bf16_tiled_weights(_bf16(w13[:4], gpu), _bf16(w2[:4], gpu),
                                                                _bf16(w13[4], gpu), _bf16(w2[4], gpu))
    ids = ids % 4
    xt = _bf16(x, gpu)
    a = moe.fused_moe_bf16_tiled_with_shared(xt, prepared, torch.from_numpy(w).to(gpu),
                                             torch.from_numpy(ids).to(gpu), routed_scaling_factor=2.5)
    ids_c = torch.from_numpy(np.concatenate([ids, np.full((19, 1), 4)], 1).astype(np.int64)).to(gpu)
    w_c = torch.from_numpy(np.concatenate([w * np.float32(2.5), np.ones((19, 1), np.float32)], 1)).to(gpu)
    b = moe.fused_moe_bf16_tiled(xt, prepared.packed, w_c, ids_c)
    assert torch.equal(a, b)


@pytest.mark.parametrize("T,Hd,F,activation,bias", [(1, 7168, 2048, "silu", False), (17, 200, 72, "gelu", True),
                                                    (64, 7168, 2048, "silu", True), (40, 96, 40, "silu", False),
                                                    (97, 1000, 300, "gelu", True), (128, 7168, 2048, "silu", False),
                                                    (200, 7168, 2048, "silu", True), (256, 520, 130, "gelu", False)])
def test_bf16_single_expert_small_rows_within_tolerance(gpu, oracle_lib, monkeypatch, T, Hd, F, activation, bias):
    """One packed expert and at most 256 routes run both GEMMs on the small-M
    kernel (split K, fp32 partial sums added in split order, the activation
    and route stores in the reduce launches): the shared MLP and a one-expert
    MoE against the fp32 reference, with biases, ragged H/F (zero-padded K),
    and out-of-range ids with the id check off (dropped by the route build,
    contributing nothing: the kernel sees fewer routed rows than routes). With
    one route per token the W2 reduce launch also merges it (no combine
    launch), skip_weighted included."""
    from fused_cpp_amd import moe

    rng = np.random.default_rng(T * 31 + Hd)
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((1, 2 * F, Hd)) * 0.02).astype(np.float32)))
    w2 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((1, Hd, F)) * 0.02).astype(np.float32)))
    b13 = (rng.standard_normal((1, 2 * F)) * 0.1).astype(np.float32) if bias else None
    b2 = (rng.standard_normal((1, Hd)) * 0.1).astype(np.float32) if bias else None
    tb = lambda a: torch.from_numpy(a).to(gpu) if a is not None else None  # noqa: E731
    packed = moe.prepare_fused_moe_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu))
    w = rng.random((T, 1)).astype(np.float32) + 0.5
    ids = np.zeros((T, 1), np.int32)
    out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, tb(w), tb(ids), w13_bias=tb(b13), w2_bias=tb(b2),
                                   activation=activation)
    ref = oracle_lib.bf16_moe_reference(x, w13, w2, w, ids, w13_bias=b13, w2_bias=b2, activation=activation,
                                        round_intermediate=True)
    _close(out, ref)
    if activation == "silu" and not bias:
        sm = moe.prepare_shared_mlp_bf16_tiled_weights(_bf16(w13[0], gpu), _bf16(w2[0], gpu))
        one = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, torch.ones((T, 1), device=gpu),
                                       torch.zeros((T, 1), dtype=torch.int32, device=gpu))
        assert torch.equal(moe.shared_mlp_bf16_tiled(_bf16(x, gpu), sm), one)
    if T > 2:
        ids[::3] = 1  # out of range: dropped
        monkeypatch.setenv("FUSED_CPP_AMD_VALIDATE_IDS", "0")
        out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, tb(w), tb(ids), w13_bias=tb(b13), w2_bias=tb(b2),
                                       activation=activation)
        keep = ids[:, 0] == 0
        ref = oracle_lib.bf16_moe_reference(x[keep], w13, w2, w[keep], ids[keep], w13_bias=b13, w2_bias=b2,
                                            activation=activation, round_intermediate=True)
        got = out.float().cpu().numpy()
        assert not got[~keep].any()
        _close(out[torch.from_numpy(np.nonzero(keep)[0]).to(gpu)], ref)
        # skip_weighted: the route row itself, the weights ignored
        out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, tb(w), tb(ids), w13_bias=tb(b13), w2_bias=tb(b2),
                                       activation=activation, skip_weighted=True)
        ref = oracle_lib.bf16_moe_reference(x[keep], w13, w2, w[keep], ids[keep], w13_bias=b13, w2_bias=b2,
                                            activation=activation, skip_weighted=True, round_intermediate=True)
        assert not out.float().cpu().numpy()[~keep].any()
        _close(out[torch.from_numpy(np.nonzero(keep)[0]).to(gpu)], ref)


@pytest.mark.parametrize("rows,hd,f", [(1, 192, 96), (13, 192, 96), (97, 192, 96), (50, 200, 72), (300, 192, 96)])
def test_shared_mlp_equals_one_expert_moe(gpu, rows, hd, f):
    """tests/test_shared_mlp_bf16_tiled.py:37-71: exact. Up to 256 rows the
    shared MLP runs no route build (row t, weight 1) and the one-expert MoE
    does: equal bit for bit, also with H not a multiple of 32 (padded rows);
    300 rows take the tiled path."""
    from fused_cpp_amd import moe

    rng = np.random.default_rng(20260816 + rows)
    x = rng.standard_normal((rows, hd)).astype(np.float32) * 0.01
    w13 = rng.standard_normal((2 * f, hd)).astype(np.float32) * 0.01
    w2 = rng.standard_normal((hd, f)).astype(np.float32) * 0.01
    packed = moe.prepare_shared_mlp_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu))
    xt = _bf16(x, gpu)
    cand = moe.shared_mlp_bf16_tiled(xt, packed, num_threads=8)
    ref = moe.fused_moe_bf16_tiled(xt, packed, torch.ones((rows, 1), device=gpu),
                                   torch.zeros((rows, 1), dtype=torch.int32, device=gpu))
    assert torch.equal(cand, ref)
    out = torch.empty_like(xt)
    assert moe.shared_mlp_bf16_tiled(xt, packed, out=out) is out and torch.equal(out, ref)


# ----------------------------------------------------------------- i8gemm --

@pytest.mark.parametrize("m,k,n,out_dtype", [(1, 7, 5, torch.float32), (4, 16, 8, torch.bfloat16),
                                             (9, 31, 13, torch.bfloat16), (24, 64, 96, torch.float32),
                                             (24, 64, 96, torch.bfloat16), (300, 7168, 512, torch.bfloat16),
                                             (520, 2048, 1000, torch.float32),
                                             (2048, 100, 8448, torch.bfloat16), (200, 640, 1001, torch.bfloat16),
                                             (1000, 300, 998, torch.float32), (300, 3000, 700, torch.float32),
                                             (700, 8192, 520, torch.bfloat16), (257, 4096, 300, torch.bfloat16)])
def test_i8gemm_bit_exact(gpu, oracle_lib, m, k, n, out_dtype):
    """tests/test_i8gemm.py:40-94 shapes (+ a DSv3-width projection; 256-row
    tiles on 256-channel workgroups with a ragged last row tile and channel
    block (520 rows); and 2048 x 8448, which on 256 CUs needs one round of
    256 x 384 workgroups against two of 256 x 256 and takes the former; the
    epilogue's 16-byte row pieces and its channel-by-channel fallback for row
    strides that are not a multiple of the piece (1001, 998 channels); and K
    split over the grid where the items fill few CUs (300 rows: 7 splits; 520:
    2; 300 rows at 47 chunks: 2 splits, the last of odd length; 700 rows: 16;
    257 rows: 4 splits, the second row tile one row),
    int32 partial sums reduced in split order)."""
    from fused_cpp_amd import i8gemm

    torch.manual_seed(0)
    weight = torch.randint(-16, 17, (n, k), dtype=torch.int8)
    weight_scale = torch.rand(n, dtype=torch.float32) * 0.05 + 0.01
    bias = torch.randn(n, dtype=torch.bfloat16)
    x = torch.randn(m, k, dtype=torch.bfloat16)
    packed = i8gemm.prepare(weight, weight_scale)
    out = i8gemm.dynamic_scaled_mm(x.to(gpu), packed, bias=bias.to(gpu), out_dtype=out_dtype)
    assert out.shape == (m, n) and out.dtype == out_dtype
    ref = oracle_lib.i8gemm(x.view(torch.int16).numpy().view(np.uint16), weight.numpy(), weight_scale.numpy(),
                            bias.float().numpy(), out_dtype == torch.bfloat16)
    got = out.cpu()
    if out_dtype == torch.bfloat16:
        np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), ref)
    else:
        np.testing.assert_array_equal(got.numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("m,k,n,bias,out_dtype", [
    (1, 64, 16, True, torch.bfloat16),      # one row, one chunk, one tile
    (7, 1000, 100, True, torch.float32),    # ragged K (padded chunk) and N (partial tile and workgroup)
    (16, 8192, 1000, False, torch.bfloat16),  # K split 16 ways (partial sums + reduce launch)
    (33, 1536, 4096, True, torch.bfloat16),   # three row fragments, a few splits
    (64, 8192, 7168, False, torch.bfloat16),  # wo_b-like width, 5 splits
    (64, 2048, 24576, False, torch.float32),  # many channel groups, one split
    (65, 3000, 700, True, torch.float32),     # five row fragments (the 8-fragment kernel, rows past m)
    (100, 7168, 2048, False, torch.bfloat16),
    (128, 16384, 1024, True, torch.bfloat16),
    (129, 5000, 300, False, torch.float32),   # 16 row fragments: two A loads per wave and chunk
    (256, 16384, 7168, True, torch.bfloat16),  # the largest small-M product
])
def test_i8gemm_small_m_split_k_bit_exact(gpu, oracle_lib, m, k, n, bias, out_dtype):
    """i8gemm at <= 256 rows runs the small-M kernel (all rows per wave, K split
    over the grid with int32 partial sums): bit-exact against the oracle, with
    extreme int8 values and rows of zeros (scale 1)."""
    from fused_cpp_amd import i8gemm

    g = torch.Generator().manual_seed(m * 7 + k + n)
    weight = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    weight[0, :] = -128
    weight_scale = torch.rand(n, dtype=torch.float32, generator=g) * 0.01 + 0.001
    b = torch.randn(n, dtype=torch.float32, generator=g) if bias else None
    x = (torch.randn(m, k, generator=g) * 3).to(torch.bfloat16)
    x[0, : min(k, 5)] = 127.0
    if m > 2:
        x[2] = 0.0
    packed = i8gemm.prepare(weight, weight_scale)
    out = i8gemm.dynamic_scaled_mm(x.to(gpu), packed, bias=b.to(gpu) if bias else None, out_dtype=out_dtype)
    ref = oracle_lib.i8gemm(x.view(torch.int16).numpy().view(np.uint16), weight.numpy(), weight_scale.numpy(),
                            b.numpy() if bias else None, out_dtype == torch.bfloat16)
    got = out.cpu()
    if out_dtype == torch.bfloat16:
        np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), ref)
    else:
        np.testing.assert_array_equal(got.numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kind", ["bf16", "w8a16"])
def test_forward_activation_rows_beyond_2gib(gpu, oracle_lib, kind):
    """Maximum sizes: 150000 x 7168 bf16 token rows (2.15 GB) exceed the 2 GiB a
    32-bit buffer offset reaches. BF16's W13 then runs its 128-256-row tiles on
    the 64-bit-addressed register kernel, and W8A16 keeps to its 16/32-row
    classes. Tokens before, across and after the boundary are checked against
    the fp32 reference (tokens are independent, so the reference only needs
    the sampled ones), within max-abs 2e-2 and cosine 0.9999."""
    from fused_cpp_amd import moe

    T, Hd, F, E = 150000, 7168, 64, 2
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    x = torch.randn(T, Hd, dtype=torch.bfloat16, device=gpu, generator=g)
    rng = np.random.default_rng(6)
    w13 = H.bf16_bits((rng.standard_normal((E, 2 * F, Hd)) * 0.02).astype(np.float32))
    w2 = H.bf16_bits((rng.standard_normal((E, Hd, F)) * 0.02).astype(np.float32))
    ids = rng.integers(0, E, size=(T, 1)).astype(np.int64)
    w = np.ones((T, 1), np.float32)
    wt, it = torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu)
    tb = lambda b: torch.from_numpy(b.view(np.int16)).to(gpu).view(torch.bfloat16)  # noqa: E731
    if kind == "bf16":
        packed = moe.prepare_fused_moe_bf16_tiled_weights(tb(w13), tb(w2))
        out = moe.fused_moe_bf16_tiled(x, packed, wt, it)
        d13, d2, rnd = H.bits_to_f32(w13), H.bits_to_f32(w2), False
    else:
        q13, s13 = oracle_lib.quant_weight_rows(w13)
        q2, s2 = oracle_lib.quant_weight_rows(w2)
        packed = moe.prepare_fused_moe_w8a16_tiled_quantized_weights(torch.from_numpy(q13), torch.from_numpy(s13),
                                                                      torch.from_numpy(q2), torch.from_numpy(s2))
        out = moe.fused_moe_w8a16_tiled(x, packed, wt, it)
        d13 = q13.astype(np.float32) * s13[..., None]
        d2 = q2.astype(np.float32) * s2[..., None]
        rnd = True
    boundary = (1 << 31) // (Hd * 2)
    rows = np.r_[0:4, boundary - 4:boundary + 4, T - 4:T]
    idx = torch.from_numpy(rows).to(gpu)
    xs = x.index_select(0, idx).float().cpu().numpy()
    ref = oracle_lib.bf16_moe_reference(xs, d13, d2, w[rows], ids[rows], round_intermediate=rnd).astype(np.float64)
    o = out.index_select(0, idx).float().cpu().numpy().astype(np.float64)
    err = float(np.abs(o - ref).max())
    cos = float((o * ref).sum() / np.sqrt((o * o).sum() * (ref * ref).sum()))
    assert err <= 2e-2 * max(1.0, float(np.abs(ref).max())), err
    assert cos >= 0.9999, cos


def test_i8gemm_activation_rows_beyond_2gib(gpu, oracle_lib):
    """Maximum sizes: 320000 x 7168 int8 activation rows (2.29 GB) exceed the
    2 GiB a 32-bit buffer offset reaches, so the 256-row tiles run on the
    64-bit-addressed kernel. Rows before, across and after the 2 GiB boundary
    are checked bit for bit (row quantisation is per row, so the oracle only
    needs the sampled rows)."""
    from fused_cpp_amd import i8gemm

    m, k, n = 320000, 7168, 32
    g = torch.Generator(device=gpu)
    g.manual_seed(3)
    x = torch.randn(m, k, dtype=torch.bfloat16, device=gpu, generator=g)
    torch.manual_seed(4)
    weight = torch.randint(-127, 128, (n, k), dtype=torch.int8)
    weight_scale = torch.rand(n, dtype=torch.float32) * 0.05 + 0.01
    out = i8gemm.dynamic_scaled_mm(x, i8gemm.prepare(weight, weight_scale), out_dtype=torch.bfloat16)
    boundary = (1 << 31) // k
    rows = np.r_[0:8, boundary - 8:boundary + 8, m - 8:m]
    idx = torch.from_numpy(rows).to(gpu)
    xs = x.index_select(0, idx).cpu().view(torch.int16).numpy().view(np.uint16)
    ref = oracle_lib.i8gemm(xs, weight.numpy(), weight_scale.numpy(), None, True)
    got = out.index_select(0, idx).cpu().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, ref)


def test_i8gemm_batched_scalar_scale_and_ties(gpu, oracle_lib):
    from fused_cpp_amd import i8gemm

    torch.manual_seed(1)
    weight = torch.randint(-8, 9, (11, 19), dtype=torch.int8)
    x = torch.randn(2, 3, 19, dtype=torch.float32)
    packed = i8gemm.prepare(weight, torch.tensor(0.02))
    out = i8gemm.dynamic_scaled_mm(x.to(gpu), packed, out_dtype=torch.bfloat16)
    assert out.shape == (2, 3, 11)
    ref = oracle_lib.i8gemm(x.reshape(6, 19).numpy(), weight.numpy(), np.float32(0.02), None, True)
    np.testing.assert_array_equal(out.cpu().reshape(6, 11).view(torch.int16).numpy().view(np.uint16), ref)
    # ties to even (tests/test_deepseek_v4_w8a8.py:40-50)
    xt = torch.zeros((2, 16), dtype=torch.bfloat16)
    xt[0, :5] = torch.tensor([127.0, 0.5, 1.5, -0.5, -1.5], dtype=torch.bfloat16)
    w = torch.zeros((8, 16), dtype=torch.int8)
    w[:5, :5] = torch.eye(5, dtype=torch.int8)
    p = i8gemm.prepare(w, torch.ones(8))
    got = i8gemm.dynamic_scaled_mm(xt.to(gpu), p, out_dtype=torch.float32).cpu()
    assert got[0, :5].tolist() == [127.0, 0.0, 2.0, 0.0, -2.0]
    a, b = i8gemm.dynamic_scaled_mm_pair(xt.to(gpu), p, p)
    assert torch.equal(a, b)


@pytest.mark.parametrize("activation", ["silu", "swigluoai"])
def test_bf16_prefill_every_tile_class_within_tolerance(gpu, oracle_lib, activation):
    """Per-expert counts 3..420 reach every prefill tile class (16, 128, 192 and
    256 rows, the last with a two-tile expert), i.e. the bf16 instantiations of
    the register-ring kernel and of the LDS-staged prefill kernel, with biases,
    against the fp32 reference."""
    from fused_cpp_amd import moe

    rng = np.random.default_rng(17)
    counts = [3, 20, 40, 70, 100, 150, 200, 260, 420]
    E, Hd, F = len(counts), 256, 192
    T = sum(counts)
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E, 2 * F, Hd)) * 0.05).astype(np.float32)))
    w2 = H.bits_to_f32(H.bf16_bits((rng.standard_normal((E, Hd, F)) * 0.05).astype(np.float32)))
    b13 = (rng.standard_normal((E, 2 * F)) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal((E, Hd)) * 0.1).astype(np.float32)
    ids = rng.permutation(np.concatenate([np.full(c, e) for e, c in enumerate(counts)])).reshape(-1, 1).astype(np.int64)
    w = np.ones((T, 1), np.float32)
    packed = moe.prepare_fused_moe_bf16_tiled_weights(_bf16(w13, gpu), _bf16(w2, gpu),
                                                      fuse_silu=activation == "silu")
    out = moe.fused_moe_bf16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu),
                                   w13_bias=torch.from_numpy(b13).to(gpu), w2_bias=torch.from_numpy(b2).to(gpu),
                                   activation=activation)
    ref = oracle_lib.bf16_moe_reference(x, w13, w2, w, ids, w13_bias=b13, w2_bias=b2, activation=activation,
                                        round_intermediate=True)
    _close(out, ref)
