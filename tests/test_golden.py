"""Committed known-answer fixtures (tests/golden/, made by make_golden.py)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

GOLD = Path(__file__).resolve().parent / "golden"


def test_oracle_reproduces_w8a8_fixture(oracle_lib):
    d = np.load(GOLD / "w8a8_ref_case.npz")
    bits = oracle_lib.w8a8_forward(d["x_bits"], d["ids"], d["w"], d["q13"], d["s13"], d["q2"], d["s2"])
    np.testing.assert_array_equal(bits, d["expect_bits"])
    f = lambda b: torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float()  # noqa: E731
    torch.testing.assert_close(f(bits), f(d["expect_formula"]), rtol=0.0, atol=3.0e-6)


def test_oracle_reproduces_i8gemm_fixtures(oracle_lib):
    d = np.load(GOLD / "i8gemm_ref_cases.npz")
    for i in range(3):
        out = d[f"o{i}"]
        got = oracle_lib.i8gemm(d[f"x{i}"], d[f"w{i}"], d[f"s{i}"], d[f"b{i}"], out.dtype == np.uint16)
        np.testing.assert_array_equal(got.view(np.uint32) if got.dtype == np.float32 else got,
                                      out.view(np.uint32) if out.dtype == np.float32 else out)


@pytest.mark.gpu
def test_gpu_reproduces_w8a8_fixture(gpu):
    from tests import helpers as H

    d = np.load(GOLD / "w8a8_ref_case.npz")
    out = H.gpu_w8a8_forward(d["x_bits"], d["ids"], d["w"], d["q13"], d["s13"], d["q2"], d["s2"], gpu)
    np.testing.assert_array_equal(out, d["expect_bits"])


@pytest.mark.gpu
def test_gpu_reproduces_i8gemm_fixtures(gpu):
    from fused_cpp_amd import i8gemm

    d = np.load(GOLD / "i8gemm_ref_cases.npz")
    for i in range(3):
        out = d[f"o{i}"]
        bf16 = out.dtype == np.uint16
        p = i8gemm.prepare(torch.from_numpy(d[f"w{i}"]), torch.from_numpy(d[f"s{i}"]))
        x = torch.from_numpy(d[f"x{i}"].view(np.int16)).view(torch.bfloat16).to(gpu)
        got = i8gemm.dynamic_scaled_mm(x, p, bias=torch.from_numpy(d[f"b{i}"]).to(gpu),
                                       out_dtype=torch.bfloat16 if bf16 else torch.float32).cpu()
        if bf16:
            np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), out)
        else:
            np.testing.assert_array_equal(got.numpy().view(np.uint32), out.view(np.uint32))
