# -*- coding: utf-8 -*-
"""Dynamic per-row W8A8 linear on MI355X: the ``fused_cpp.i8gemm`` surface
(src/fused_cpp/i8gemm.py).

    packed = i8gemm.prepare(weight_int8, weight_scale)
    out = i8gemm.dynamic_scaled_mm(x, packed, bias=None, out_dtype=torch.bfloat16)

Semantics (csrc/i8gemm.cpp:368-392 and :148-164, pinned by the reference's
tests/test_i8gemm.py:18-37): per row scale = max|x|/127 (1 if zero),
q = rint(x / scale) (ties to even) clamped to [-128, 127], int32 GEMM on
int8 MFMA, out = acc * x_scale * w_scale[n] (+ bias) in fp32, then cast.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from fused_cpp_amd import _native

_supports_i8gemm = _native.moe_C is not None and _native.gpu_available()
_i8gemm_dynamic_scaled_mm_pair = getattr(_native.moe_C, "i8gemm_dynamic_scaled_mm_pair", None)


def _require_backend() -> None:
    _native.require_native()
    if not _native.gpu_available():
        raise RuntimeError("i8gemm backend unavailable: no ROCm device is visible")


@dataclass(frozen=True)
class PreparedI8GEMMWeight:
    """Packed int8 linear weight (``[N, K]`` vLLM layout before packing) and metadata."""

    packed_weight: torch.Tensor
    weight_scale: torch.Tensor
    k: int
    n: int
    k_padded: int
    n_padded: int
    backend: str


def prepare(weight_int8: torch.Tensor, weight_scale: torch.Tensor, *, backend: str = "auto") -> PreparedI8GEMMWeight:
    """Prepare an int8 ``[N, K]`` weight for repeated GEMMs (i8gemm.py:58-85)."""
    _require_backend()
    if weight_int8.dim() != 2:
        raise RuntimeError(f"i8gemm.prepare: weight_int8 must be 2D [N, K], got {weight_int8.dim()}D")
    if weight_int8.dtype != torch.int8:
        raise RuntimeError(f"i8gemm.prepare: weight_int8 dtype must be torch.int8, got {weight_int8.dtype}")
    if weight_scale.numel() not in (1, int(weight_int8.shape[0])):
        raise RuntimeError("i8gemm.prepare: weight_scale must be scalar or shape [N]")
    dev = torch.device("cuda", torch.cuda.current_device()) if weight_int8.device.type != "cuda" else weight_int8.device
    packed, scale, k, n, kp, np_, selected = _native.moe_C.i8gemm_prepare(
        weight_int8.to(dev).contiguous(), weight_scale.to(dev).contiguous())
    return PreparedI8GEMMWeight(packed_weight=packed, weight_scale=scale, k=int(k), n=int(n), k_padded=int(kp),
                                n_padded=int(np_), backend=str(selected))


def _i8gemm_dynamic_scaled_mm(out, x, packed_weight, weight_scale, bias, k, n, kp=None, np_=None, nthreads=0):
    """Direct native call (the reference's ``_C.i8gemm_dynamic_scaled_mm`` argument order)."""
    _native.moe_C.i8gemm_dynamic_scaled_mm(out, x, packed_weight, weight_scale, bias, int(k), int(n))


def dynamic_scaled_mm(
    x: torch.Tensor,
    packed: PreparedI8GEMMWeight,
    *,
    bias: Optional[torch.Tensor] = None,
    out_dtype: torch.dtype = torch.bfloat16,
    nthreads: int = 0,
) -> torch.Tensor:
    """``x @ weight.T`` with dynamic per-token int8 quantisation (i8gemm.py:88-137)."""
    _require_backend()
    if not isinstance(packed, PreparedI8GEMMWeight):
        raise RuntimeError("i8gemm.dynamic_scaled_mm: packed must come from i8gemm.prepare")
    if x.shape[-1] != packed.k:
        raise RuntimeError(f"i8gemm.dynamic_scaled_mm: x last dim must be K={packed.k}, got {x.shape[-1]}")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"i8gemm.dynamic_scaled_mm: x dtype must be float32/bfloat16, got {x.dtype}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"i8gemm.dynamic_scaled_mm: out_dtype must be float32/bfloat16, got {out_dtype}")
    if x.device.type != "cuda":
        raise RuntimeError("i8gemm.dynamic_scaled_mm: x must be a ROCm device tensor")
    if bias is not None:
        if bias.dim() != 1 or int(bias.shape[0]) != packed.n:
            raise RuntimeError(f"i8gemm.dynamic_scaled_mm: bias must be shape [{packed.n}]")
        bias = bias.contiguous()
    batch_shape = tuple(x.shape[:-1])
    out_shape = (*batch_shape, packed.n)
    if x.numel() == 0:
        return torch.empty(out_shape, dtype=out_dtype, device=x.device)
    x_2d = x.contiguous().reshape(-1, packed.k)
    out_2d = torch.empty((x_2d.shape[0], packed.n), dtype=out_dtype, device=x.device)
    _native.moe_C.i8gemm_dynamic_scaled_mm(out_2d, x_2d, packed.packed_weight, packed.weight_scale, bias, packed.k,
                                           packed.n)
    return out_2d.reshape(out_shape)


def mm(x: torch.Tensor, packed: PreparedI8GEMMWeight, *, bias: Optional[torch.Tensor] = None,
       out_dtype: torch.dtype = torch.bfloat16, nthreads: int = 0) -> torch.Tensor:
    """Alias for :func:`dynamic_scaled_mm`."""
    return dynamic_scaled_mm(x, packed, bias=bias, out_dtype=out_dtype, nthreads=nthreads)


def dynamic_scaled_mm_pair(x: torch.Tensor, first: PreparedI8GEMMWeight, second: PreparedI8GEMMWeight, *,
                           nthreads: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """Two BF16-output GEMMs sharing one dynamic per-row activation quantisation (i8gemm.py:151-189).

    The input rows are quantised once (scale = max|x|/127, ties-to-even rounding,
    csrc/i8gemm.cpp:486-505) and both GEMMs read the same int8 rows.
    """
    _require_backend()
    if _i8gemm_dynamic_scaled_mm_pair is None:
        raise RuntimeError("i8gemm dynamic pair kernel is unavailable in this build")
    if not isinstance(first, PreparedI8GEMMWeight) or not isinstance(second, PreparedI8GEMMWeight):
        raise TypeError("first and second must be PreparedI8GEMMWeight")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError("i8gemm.dynamic_scaled_mm_pair input must be BF16 [M, K]")
    if first.k != second.k or first.k_padded != second.k_padded or x.shape[1] != first.k:
        raise ValueError("paired i8gemm weights and input must share K and Kp")
    if int(nthreads) < 0:
        raise ValueError("nthreads must be non-negative; zero selects the backend default")
    x = x.to(first.packed_weight.device).contiguous()
    first_output = torch.empty((x.shape[0], first.n), dtype=torch.bfloat16, device=x.device)
    second_output = torch.empty((x.shape[0], second.n), dtype=torch.bfloat16, device=x.device)
    _i8gemm_dynamic_scaled_mm_pair(first_output, second_output, x, first.packed_weight, first.weight_scale,
                                   int(first.k), int(first.n), second.packed_weight, second.weight_scale,
                                   int(second.n))
    return first_output, second_output


__all__ = [
    "PreparedI8GEMMWeight",
    "_supports_i8gemm",
    "dynamic_scaled_mm",
    "dynamic_scaled_mm_pair",
    "mm",
    "prepare",
]
