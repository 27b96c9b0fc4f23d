"""Regenerate tests/golden/*.npz (small known-answer fixtures).

w8a8_ref_case.npz: the exact inputs of the reference test
  tests/test_moe_w8a8.py:197-226 (torch.Generator seed 23, H=F=64, T=48,
  2 experts, top-1), with
  - expect_formula: that test's own per-token reference formula
    (tests/test_moe_w8a8.py:40-69; the reference kernel matches it to 3e-6),
  - expect_bits: this repository's oracle output (bit pattern the GPU must
    reproduce).
i8gemm_ref_cases.npz: tests/test_i8gemm.py:40-58 inputs (torch.manual_seed(0))
  with outputs of that test's closed form (atol 0 in the reference).

Run from the repo root: python -m tests.golden.make_golden
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def w8a8_case():
    from tests.test_oracle_pins import _reference_moe_w8a8

    import oracle

    g = torch.Generator().manual_seed(23)
    experts, hidden, inter, tokens = 2, 64, 64, 48
    q13 = torch.randint(-12, 13, (experts, 2 * inter, hidden), dtype=torch.int8, generator=g)
    q2 = torch.randint(-12, 13, (experts, hidden, inter), dtype=torch.int8, generator=g)
    s13 = torch.rand((experts, 2 * inter), generator=g) * 0.003 + 0.0005
    s2 = torch.rand((experts, hidden), generator=g) * 0.003 + 0.0005
    x = (torch.randn((tokens, hidden), generator=g) * 0.3).to(torch.bfloat16)
    ids = torch.tensor([[t % experts] for t in range(tokens)], dtype=torch.int64)
    w = torch.ones((tokens, 1), dtype=torch.float32)
    formula = _reference_moe_w8a8(x, q13, s13, q2, s2, w, ids)
    x_bits = x.view(torch.int16).numpy().view(np.uint16)
    bits = oracle.w8a8_forward(x_bits, ids.numpy(), w.numpy(), q13.numpy(), s13.numpy(), q2.numpy(), s2.numpy())
    np.savez(HERE / "w8a8_ref_case.npz", x_bits=x_bits, ids=ids.numpy(), w=w.numpy(), q13=q13.numpy(),
             s13=s13.numpy(), q2=q2.numpy(), s2=s2.numpy(),
             expect_formula=formula.view(torch.int16).numpy().view(np.uint16), expect_bits=bits)


def i8gemm_cases():
    from tests.test_oracle_pins import _reference_i8gemm

    arrays = {}
    torch.manual_seed(0)
    for i, (m, k, n, bf16) in enumerate([(1, 7, 5, False), (4, 16, 8, True), (9, 31, 13, True)]):
        weight = torch.randint(-16, 17, (n, k), dtype=torch.int8)
        scale = torch.rand(n, dtype=torch.float32) * 0.05 + 0.01
        bias = torch.randn(n, dtype=torch.bfloat16)
        x = torch.randn(m, k, dtype=torch.bfloat16)
        out = _reference_i8gemm(x, weight, scale, bias=bias, out_dtype=torch.bfloat16 if bf16 else torch.float32)
        arrays[f"x{i}"] = x.view(torch.int16).numpy().view(np.uint16)
        arrays[f"w{i}"] = weight.numpy()
        arrays[f"s{i}"] = scale.numpy()
        arrays[f"b{i}"] = bias.float().numpy()
        arrays[f"o{i}"] = (out.view(torch.int16).numpy().view(np.uint16) if bf16 else out.numpy())
    np.savez(HERE / "i8gemm_ref_cases.npz", **arrays)


if __name__ == "__main__":
    w8a8_case()
    i8gemm_cases()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
