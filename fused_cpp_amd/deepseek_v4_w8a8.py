# -*- coding: utf-8 -*-
"""W8A8 linears for DeepSeek V4 attention projections on MI355X: the
``fused_cpp.deepseek_v4_w8a8`` surface (src/fused_cpp/deepseek_v4_w8a8.py).

Weights are quantised per output channel (scale = max|w|/127, or 1 for an
all-zero row; q = round-half-even(w / scale) clamped to +-127,
deepseek_v4_w8a8.py:44-53) on the GPU and packed once. The linears run
``fused_cpp_amd.i8gemm`` (dynamic per-row activation quantisation, int8
MFMA, channel dequant, bf16 store); ``deepseek_v4_w8a8_linear_pair`` shares one
activation quantisation between the main and indexer Q projections
(:114-132).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from fused_cpp_amd import cabi, i8gemm

_HAS_DEEPSEEK_V4_W8A8 = bool(i8gemm._supports_i8gemm)


@dataclass(frozen=True)
class PreparedDeepSeekV4W8A8LinearWeight:
    """Opaque per-output-channel W8 weight for dynamic per-row A8 GEMM."""

    packed: i8gemm.PreparedI8GEMMWeight

    @property
    def k(self) -> int:
        return self.packed.k

    @property
    def n(self) -> int:
        return self.packed.n


def _device(t: torch.Tensor) -> torch.Tensor:
    return t if t.device.type == "cuda" else t.to(torch.device("cuda", torch.cuda.current_device()))


def _quantize_weight_per_output_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if weight.dtype != torch.bfloat16:
        raise TypeError("DeepSeek V4 W8A8 source weight must be a torch.bfloat16 tensor")
    if weight.dim() != 2:
        raise ValueError(f"DeepSeek V4 W8A8 source weight must be [N, K], got {tuple(weight.shape)}")
    w = _device(weight).contiguous()
    n, k = w.shape
    q = torch.empty((n, k), dtype=torch.int8, device=w.device)
    s = torch.empty((n,), dtype=torch.float32, device=w.device)
    cabi.check(cabi.lib().fcmoe_quantize_weight_rows(w.data_ptr(), n, k, q.data_ptr(), s.data_ptr(),
                                                     cabi.stream_handle()), "quantize_weight_rows")
    return q, s


def prepare_deepseek_v4_w8a8_linear_weight(weight: torch.Tensor, *, backend: str = "auto"
                                           ) -> PreparedDeepSeekV4W8A8LinearWeight:
    """Quantize one BF16 ``[N, K]`` attention weight and pack it once."""
    i8gemm._require_backend()
    quantized, scale = _quantize_weight_per_output_channel(weight)
    return prepare_deepseek_v4_w8a8_linear_quantized_weight(quantized, scale, backend=backend)


def prepare_deepseek_v4_w8a8_linear_quantized_weight(weight: torch.Tensor, scale: torch.Tensor, *,
                                                     backend: str = "auto") -> PreparedDeepSeekV4W8A8LinearWeight:
    """Pack checkpoint INT8 ``[N, K]`` weight with FP32 channel scales."""
    if weight.dtype != torch.int8 or weight.dim() != 2:
        raise TypeError("DeepSeek V4 quantized weight must be a torch.int8 [N, K] tensor")
    if scale.dtype != torch.float32:
        raise TypeError("DeepSeek V4 W8 scale must be a torch.float32 tensor")
    if scale.numel() != weight.shape[0]:
        raise ValueError(f"DeepSeek V4 W8 scale must contain N={weight.shape[0]} values")
    return PreparedDeepSeekV4W8A8LinearWeight(
        packed=i8gemm.prepare(weight.contiguous(), scale.reshape(-1).contiguous(), backend=backend))


def deepseek_v4_w8a8_linear(input: torch.Tensor, weight: PreparedDeepSeekV4W8A8LinearWeight, *,
                            num_threads: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """Dynamic A8 quantization, int8 GEMM, channel dequant and BF16 store (deepseek_v4_w8a8.py:84-111)."""
    if not isinstance(weight, PreparedDeepSeekV4W8A8LinearWeight):
        raise TypeError("weight must be PreparedDeepSeekV4W8A8LinearWeight")
    if input.dtype != torch.bfloat16:
        raise TypeError("DeepSeek V4 W8A8 input must be a torch.bfloat16 tensor")
    if input.shape[-1] != weight.k:
        raise ValueError(f"DeepSeek V4 W8A8 input K must be {weight.k}, got {input.shape[-1]}")
    if int(num_threads) < 0:
        raise ValueError("num_threads must be non-negative; zero selects the backend default")
    result = i8gemm.dynamic_scaled_mm(input, weight.packed, out_dtype=torch.bfloat16, nthreads=int(num_threads))
    if out is None:
        return result
    if out.device != result.device or out.dtype != result.dtype or out.shape != result.shape or not out.is_contiguous():
        raise ValueError("out must be contiguous BF16 with shape [*, N] on the input's device")
    out.copy_(result)
    return out


def deepseek_v4_w8a8_linear_pair(input: torch.Tensor, first: PreparedDeepSeekV4W8A8LinearWeight,
                                 second: PreparedDeepSeekV4W8A8LinearWeight, *, num_threads: int = 0
                                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """Main/indexer Q projections with one shared activation quantization (deepseek_v4_w8a8.py:114-132)."""
    if not isinstance(first, PreparedDeepSeekV4W8A8LinearWeight) or not isinstance(
            second, PreparedDeepSeekV4W8A8LinearWeight):
        raise TypeError("paired weights must be PreparedDeepSeekV4W8A8LinearWeight")
    if input.dtype != torch.bfloat16 or input.dim() != 2:
        raise TypeError("DeepSeek V4 paired W8A8 input must be BF16 [M, K]")
    if first.k != second.k or input.shape[1] != first.k:
        raise ValueError("paired W8A8 weights and input must share K")
    if int(num_threads) < 0:
        raise ValueError("num_threads must be non-negative; zero selects the backend default")
    return i8gemm.dynamic_scaled_mm_pair(input, first.packed, second.packed, nthreads=int(num_threads))


def deepseek_v4_wo_b_w8a8(input: torch.Tensor, weight: PreparedDeepSeekV4W8A8LinearWeight, *,
                          num_threads: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """The TP-local ``attn.wo_b`` projection; the collective reduction stays external (:135-143)."""
    return deepseek_v4_w8a8_linear(input, weight, num_threads=num_threads, out=out)


__all__ = [
    "PreparedDeepSeekV4W8A8LinearWeight",
    "_HAS_DEEPSEEK_V4_W8A8",
    "deepseek_v4_w8a8_linear",
    "deepseek_v4_w8a8_linear_pair",
    "deepseek_v4_wo_b_w8a8",
    "prepare_deepseek_v4_w8a8_linear_quantized_weight",
    "prepare_deepseek_v4_w8a8_linear_weight",
]
