"""GPU W8A8 linears for DeepSeek V4 attention (``fused_cpp_amd.deepseek_v4_w8a8``)
and the shared-quantisation i8gemm pair.

Bar: bit-exact. The expected values follow the reference tests'
dynamic-quantisation formula (tests/test_deepseek_v4_w8a8.py:19-50): per-row
scale = max|x|/127, q = round-half-even(x / scale) clamped to +-127, exact
integer GEMM, then (float)acc * x_scale * w_scale left to right and a bf16 cast.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    fp32 = x.float()
    maximum = fp32.abs().amax(dim=1, keepdim=True)
    scale = torch.where(maximum > 0, maximum / 127.0, torch.ones_like(maximum))
    return (fp32 / scale).round().clamp(-127, 127).to(torch.int64), scale


def _expected(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    q, s = _quantize_rows(x.cpu())
    acc = q @ weight.cpu().to(torch.int64).T  # exact
    return (acc.to(torch.float32) * s * weight_scale.cpu()).to(torch.bfloat16)


def test_linear_matches_dynamic_quantization_reference(gpu):
    from fused_cpp_amd.deepseek_v4_w8a8 import deepseek_v4_w8a8_linear, prepare_deepseek_v4_w8a8_linear_quantized_weight

    g = torch.Generator().manual_seed(41)
    m, k, n = 13, 64, 96
    x = (torch.randn((m, k), generator=g) * 0.2).to(torch.bfloat16)
    weight = torch.randint(-16, 17, (n, k), dtype=torch.int8, generator=g)
    weight_scale = torch.rand((n,), generator=g) * 0.004 + 0.0005
    prepared = prepare_deepseek_v4_w8a8_linear_quantized_weight(weight, weight_scale)
    actual = deepseek_v4_w8a8_linear(x.to(gpu), prepared, num_threads=2)
    assert torch.equal(actual.cpu(), _expected(x, weight, weight_scale))


def test_dynamic_quantization_uses_ties_to_even(gpu):
    from fused_cpp_amd.deepseek_v4_w8a8 import deepseek_v4_w8a8_linear, prepare_deepseek_v4_w8a8_linear_quantized_weight

    x = torch.zeros((2, 16), dtype=torch.bfloat16)
    x[0, :5] = torch.tensor([127.0, 0.5, 1.5, -0.5, -1.5], dtype=torch.bfloat16)
    weight = torch.zeros((8, 16), dtype=torch.int8)
    weight[:5, :5] = torch.eye(5, dtype=torch.int8)
    prepared = prepare_deepseek_v4_w8a8_linear_quantized_weight(weight, torch.ones(8))
    actual = deepseek_v4_w8a8_linear(x.to(gpu), prepared, num_threads=1).cpu()
    assert torch.equal(actual, _expected(x, weight, torch.ones(8)))
    assert actual[0, :5].float().tolist() == [127.0, 0.0, 2.0, 0.0, -2.0]


def test_wo_b_alias_out_and_bf16_prepare_quantises_like_the_oracle(gpu, oracle_lib):
    from fused_cpp_amd.deepseek_v4_w8a8 import (deepseek_v4_w8a8_linear, deepseek_v4_wo_b_w8a8,
                                                 prepare_deepseek_v4_w8a8_linear_weight)

    g = torch.Generator().manual_seed(43)
    x = (torch.randn((12, 64), generator=g) * 0.2).to(torch.bfloat16).to(gpu)
    weight = (torch.randn((128, 64), generator=g) * 0.02).to(torch.bfloat16)
    prepared = prepare_deepseek_v4_w8a8_linear_weight(weight)
    _, s_ref = oracle_lib.quant_weight_rows(weight.view(torch.int16).numpy().view(np.uint16))
    np.testing.assert_array_equal(prepared.packed.weight_scale.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    expected = deepseek_v4_w8a8_linear(x, prepared, num_threads=2)
    out = torch.empty_like(expected)
    actual = deepseek_v4_wo_b_w8a8(x, prepared, num_threads=2, out=out)
    assert actual is out and torch.equal(actual, expected)


@pytest.mark.parametrize("m,k,n1,n2", [(24, 64, 96, 128), (2, 64, 13, 21), (7, 7168, 1536, 512), (300, 1024, 80, 48),
                                      (40, 2048, 2048, 512), (300, 8192, 7168, 512)])
def test_pair_equals_two_single_projections(gpu, m, k, n1, n2):
    """tests/test_deepseek_v4_w8a8.py:62-96 (incl. logical N tails) plus DSv3 Q-projection widths
    (and 300 rows at K = 8192, where the two GEMMs split K 6 and 8 ways)."""
    from fused_cpp_amd.deepseek_v4_w8a8 import (deepseek_v4_w8a8_linear, deepseek_v4_w8a8_linear_pair,
                                                 prepare_deepseek_v4_w8a8_linear_quantized_weight)

    g = torch.Generator().manual_seed(m + n1)
    x = (torch.randn((m, k), generator=g) * 0.2).to(torch.bfloat16)
    w1 = torch.randint(-17, 18, (n1, k), dtype=torch.int8, generator=g)
    w2 = torch.randint(-17, 18, (n2, k), dtype=torch.int8, generator=g)
    s1 = torch.rand((n1,), generator=g) * 0.002 + 0.001
    s2 = torch.rand((n2,), generator=g) * 0.002 + 0.001
    first = prepare_deepseek_v4_w8a8_linear_quantized_weight(w1, s1)
    second = prepare_deepseek_v4_w8a8_linear_quantized_weight(w2, s2)
    a, b = deepseek_v4_w8a8_linear_pair(x.to(gpu), first, second, num_threads=2)
    assert torch.equal(a, deepseek_v4_w8a8_linear(x.to(gpu), first))
    assert torch.equal(b, deepseek_v4_w8a8_linear(x.to(gpu), second))
    assert torch.equal(a.cpu(), _expected(x, w1, s1))
    assert torch.equal(b.cpu(), _expected(x, w2, s2))


def test_pair_with_split_counts_differing_equals_singles(gpu):
    """64 rows: alone, the first GEMM (32768 channels: 256 workgroups of 8
    tiles) runs unsplit and the second (8192) splits K three ways; in the
    pair's one launch both run unsplit (320 workgroups) while (7, 7168, 1536,
    512) above splits both 14 ways. The pair equals the two single GEMMs bit
    for bit (each checked against the oracle elsewhere)."""
    from fused_cpp_amd.deepseek_v4_w8a8 import (deepseek_v4_w8a8_linear, deepseek_v4_w8a8_linear_pair,
                                                 prepare_deepseek_v4_w8a8_linear_quantized_weight)

    g = torch.Generator().manual_seed(5)
    m, k, n1, n2 = 64, 1536, 32768, 8192
    x = (torch.randn((m, k), generator=g) * 0.2).to(torch.bfloat16).to(gpu)
    first = prepare_deepseek_v4_w8a8_linear_quantized_weight(
        torch.randint(-127, 128, (n1, k), dtype=torch.int8, generator=g), torch.rand((n1,), generator=g) * 0.002 + 0.001)
    second = prepare_deepseek_v4_w8a8_linear_quantized_weight(
        torch.randint(-127, 128, (n2, k), dtype=torch.int8, generator=g), torch.rand((n2,), generator=g) * 0.002 + 0.001)
    a, b = deepseek_v4_w8a8_linear_pair(x, first, second)
    assert torch.equal(a, deepseek_v4_w8a8_linear(x, first))
    assert torch.equal(b, deepseek_v4_w8a8_linear(x, second))


def test_pair_and_linear_reject_bad_shapes(gpu):
    from fused_cpp_amd.deepseek_v4_w8a8 import (deepseek_v4_w8a8_linear, deepseek_v4_w8a8_linear_pair,
                                                 prepare_deepseek_v4_w8a8_linear_quantized_weight)

    first = prepare_deepseek_v4_w8a8_linear_quantized_weight(torch.ones((16, 32), dtype=torch.int8), torch.ones(16))
    second = prepare_deepseek_v4_w8a8_linear_quantized_weight(torch.ones((16, 48), dtype=torch.int8), torch.ones(16))
    with pytest.raises(ValueError, match="share K"):
        deepseek_v4_w8a8_linear_pair(torch.zeros((2, 32), dtype=torch.bfloat16, device=gpu), first, second)
    with pytest.raises(ValueError, match="input K"):
        deepseek_v4_w8a8_linear(torch.zeros((2, 16), dtype=torch.bfloat16, device=gpu), first)
    empty = deepseek_v4_w8a8_linear_pair(torch.zeros((0, 32), dtype=torch.bfloat16, device=gpu), first, first)
    assert empty[0].shape == (0, 16) and empty[1].shape == (0, 16)
