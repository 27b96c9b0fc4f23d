"""GPU W8A16 fused MoE (int8 per-channel weights, bf16 activations) through the
public API, against the fp32 oracle on the dequantised weights q * s.

Bar: the reference's W8A16 kernels are SVE JIT code whose rounding order
cannot be restated, so parity is a tolerance (max-abs <= 2e-2 x max(1, |ref|),
cosine >= 0.9999, the north-star BF16 bar). The oracle rounds the activation
output to bf16 as the native executors do. Weight quantisation itself
(scale = max|w|/127, q = nearbyint(w/s)) is checked bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _bf16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(H.bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)


def _close(out: torch.Tensor, ref: np.ndarray, tol: float = 2e-2, cos_min: float = 0.9999) -> None:
    o = out.float().cpu().numpy().astype(np.float64)
    r = ref.astype(np.float64)
    scale = max(1.0, float(np.abs(r).max()))
    err = float(np.abs(o - r).max())
    cos = float((o * r).sum() / np.sqrt((o * o).sum() * (r * r).sum() + 1e-300))
    assert err <= tol * scale, f"max-abs {err:.4e} > {tol} * {scale:.3f}"
    assert cos >= cos_min, f"cosine {cos:.7f} < {cos_min}"


def _case(oracle_lib, seed, T, Hd, F, E, k, w_std=0.02):
    rng = np.random.default_rng(seed)
    x = H.bits_to_f32(H.bf16_bits(rng.standard_normal((T, Hd)).astype(np.float32)))
    w13 = H.bf16_bits((rng.standard_normal((E, 2 * F, Hd)) * w_std).astype(np.float32))
    w2 = H.bf16_bits((rng.standard_normal((E, Hd, F)) * w_std).astype(np.float32))
    q13, s13 = oracle_lib.quant_weight_rows(w13)
    q2, s2 = oracle_lib.quant_weight_rows(w2)
    ids, w = H.softmax_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    deq13 = q13.astype(np.float32) * s13[..., None]
    deq2 = q2.astype(np.float32) * s2[..., None]
    return x, w13, w2, q13, s13, q2, s2, ids, w, deq13, deq2


@pytest.mark.parametrize("activation,limit", [("silu", None), ("gelu", None), ("silu", 10.0)])
@pytest.mark.parametrize("T,Hd,F,E,k", [(16, 256, 128, 8, 2), (37, 96, 40, 5, 3), (300, 128, 64, 4, 2)])
def test_w8a16_matches_dequantised_fp32_reference(gpu, oracle_lib, activation, limit, T, Hd, F, E, k):
    """Unaligned H/F (zero-padded K) and multi-tile experts (32-row class at T=300)."""
    from fused_cpp_amd import moe

    x, _, _, q13, s13, q2, s2, ids, w, deq13, deq2 = _case(oracle_lib, T * 7 + Hd, T, Hd, F, E, k)
    packed = moe.prepare_fused_moe_w8a16_tiled_quantized_weights(torch.from_numpy(q13), torch.from_numpy(s13),
                                                                  torch.from_numpy(q2), torch.from_numpy(s2))
    out = moe.fused_moe_w8a16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu),
                                    activation=activation, swiglu_limit=limit)
    act = "silu_clamp10" if limit else activation
    _close(out, oracle_lib.bf16_moe_reference(x, deq13, deq2, w, ids, activation=act, round_intermediate=True))


@pytest.mark.parametrize("activation", ["silu", "gelu"])
@pytest.mark.parametrize("T,Hd,F,E,k", [(200, 256, 128, 4, 2), (700, 200, 96, 4, 2), (900, 320, 160, 14, 2),
                                         (640, 256, 128, 8, 2)])
def test_w8a16_prefill_classes(gpu, oracle_lib, activation, T, Hd, F, E, k):
    """Prefill-sized experts on the LDS-staged W8A16 tiles: ~100 rows per
    expert (128-row class), ~350 (two 256-row tiles per expert), a mix of
    classes with unaligned H (zero-padded K) and a single-chunk W2, and ~160
    rows per expert (192-row class)."""
    from fused_cpp_amd import moe

    x, _, _, q13, s13, q2, s2, ids, w, deq13, deq2 = _case(oracle_lib, T + 3 * Hd, T, Hd, F, E, k)
    counts = np.bincount(ids.ravel(), minlength=E)
    assert counts.max() > 32  # at least one expert beyond the direct-A tiles
    packed = moe.prepare_fused_moe_w8a16_tiled_quantized_weights(torch.from_numpy(q13), torch.from_numpy(s13),
                                                                  torch.from_numpy(q2), torch.from_numpy(s2))
    out = moe.fused_moe_w8a16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu),
                                    activation=activation)
    _close(out, oracle_lib.bf16_moe_reference(x, deq13, deq2, w, ids, activation=activation, round_intermediate=True))


def test_w8a16_prepare_from_bf16_quantises_like_the_oracle(gpu, oracle_lib):
    from fused_cpp_amd import moe

    x, w13, w2, q13, s13, q2, s2, ids, w, deq13, deq2 = _case(oracle_lib, 5, 24, 512, 256, 6, 2)
    tb = lambda b: torch.from_numpy(b.view(np.int16)).to(gpu).view(torch.bfloat16)  # noqa: E731
    packed = moe.prepare_fused_moe_w8a16_tiled_weights(tb(w13), tb(w2))
    np.testing.assert_array_equal(packed.w13[3].cpu().numpy().view(np.uint32), s13.view(np.uint32))
    np.testing.assert_array_equal(packed.w2[3].cpu().numpy().view(np.uint32), s2.view(np.uint32))
    ref_packed = moe.prepare_fused_moe_w8a16_tiled_quantized_weights(
        torch.from_numpy(q13), torch.from_numpy(s13), torch.from_numpy(q2), torch.from_numpy(s2))
    assert torch.equal(packed.w13[0], ref_packed.w13[0]) and torch.equal(packed.w2[0], ref_packed.w2[0])
    assert packed.backend_name == "gfx950_w8a16_mfma"
    out = moe.fused_moe_w8a16_tiled(_bf16(x, gpu), packed, torch.from_numpy(w).to(gpu), torch.from_numpy(ids).to(gpu))
    _close(out, oracle_lib.bf16_moe_reference(x, deq13, deq2, w, ids, round_intermediate=True))


def test_w8a16_dsv3_shape_routed_shared(gpu, oracle_lib):
    """C1 shape (H=7168, I=2048) with 16 routed experts, top-8 + shared, x2.5."""
    from fused_cpp_amd import moe

    T, Hd, F, E, k = 32, 7168, 2048, 16, 8
    x, _, _, q13, s13, q2, s2, ids, w, deq13, deq2 = _case(oracle_lib, 11, T, Hd, F, E + 1, k)
    ids = np.minimum(ids, E - 1)  # routed ids only
    t = torch.from_numpy
    prepared = moe.prepare_routed_shared_moe_w8a16_tiled_quantized_weights(
        t(q13[:E]), t(s13[:E]), t(q2[:E]), t(s2[:E]), t(q13[E]), t(s13[E]), t(q2[E]), t(s2[E]))
    out = moe.fused_moe_w8a16_tiled_with_shared(_bf16(x, gpu), prepared, t(w).to(gpu), t(ids).to(gpu),
                                                routed_scaling_factor=2.5)
    ids_c = np.concatenate([ids, np.full((T, 1), E)], 1)
    w_c = np.concatenate([w * np.float32(2.5), np.ones((T, 1), np.float32)], 1)
    _close(out, oracle_lib.bf16_moe_reference(x, deq13, deq2, w_c, ids_c, round_intermediate=True))


def test_w8a16_plan_entry_dispatcher_and_errors(gpu, oracle_lib):
    from fused_cpp_amd import moe
    from fused_cpp_amd.moe.plan import AsyncMoEPlanV2

    x, _, _, q13, s13, q2, s2, ids, w, deq13, deq2 = _case(oracle_lib, 3, 9, 128, 64, 4, 2)
    t = torch.from_numpy
    packed = moe.prepare_fused_moe_w8a16_tiled_quantized_weights(t(q13), t(s13), t(q2), t(s2))
    args = (_bf16(x, gpu), packed, t(w).to(gpu), t(ids).to(gpu))
    base = moe.fused_moe_w8a16_tiled(*args)
    assert torch.equal(moe.fused_moe_tiled(*args), base)
    assert torch.equal(moe.fused_moe_tiled(*args, cache_dequant=True), base)
    out = torch.empty_like(args[0])
    assert moe.fused_moe_w8a16_tiled(*args, out=out) is out and torch.equal(out, base)
    with pytest.raises(ValueError, match="w13_bias"):
        moe.fused_moe_tiled(*args, w13_bias=torch.zeros(4, 128, device=gpu))
    with pytest.raises(ValueError):
        moe.fused_moe_w8a16_tiled(*args, activation="swigluoai")
    with pytest.raises(TypeError):
        moe.fused_moe_w8a16_tiled(args[0].float(), *args[1:])
    empty = moe.fused_moe_w8a16_tiled(args[0][:0], packed, args[2][:0], args[3][:0])
    assert empty.shape == (0, 128)
    with pytest.raises(Exception):
        moe.fused_moe_w8a16_tiled_async_plan(*args, {"bogus": 1})
    assert AsyncMoEPlanV2 is not None
