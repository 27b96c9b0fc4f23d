# -*- coding: utf-8 -*-
"""Tiled fused-MoE operators on MI355X: the drop-in surface of
``fused_cpp.moe.bf16_tiled`` (src/fused_cpp/moe/bf16_tiled.py).

Same function names, keyword arguments, defaults, prepared-weight dataclasses
and error types as the reference; tensors live on the ROCm device. Prepare
functions accept host or device weights and leave the packed result on the
current device. CPU-scheduling knobs (``num_threads``, ``thread_cpu_ids``,
plans) are accepted and validated but select nothing: the GPU operator picks
its tile shapes from the routed token counts.

Numerics (see the C ABI in include/fcmoe.h for the kernel contract):

* W8A8: per-token dynamic int8 activations (half away from zero), int8 x int8
  -> int32 MFMA, clamped SwiGLU with the reference's FEXPA exp evaluation,
  bf16 intermediate, per-row requant, int32 W2, fp32 route rows, ordered FMA
  merge -- the same binary32 operation sequence as
  csrc/moe/arm/i8mm_w8a8/kernels.cpp:200-257, 583-688.
* BF16: bf16 MFMA with fp32 accumulation, activation in fp32, bf16
  intermediate, fp32 route rows, merge as csrc/moe/arm/sve_bf16/route_merge.cpp.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Mapping, Tuple

import torch

from fused_cpp_amd import _native
from fused_cpp_amd.moe.plan import AsyncMoEPlanV2, materialize_plan

PreparedWeight = Tuple[torch.Tensor, int, int]

_BACKEND_ID = 950
_BACKEND_NAME = "gfx950_mfma"


@dataclass(frozen=True)
class PreparedBF16TiledFusedMoEWeights:
    """Packed BF16 weights (16-channel x 64-byte MFMA operand tiles)."""

    w13: PreparedWeight
    w2: PreparedWeight
    fused_silu: bool = False
    gemm_backend: int = _BACKEND_ID
    backend_n_tile: int = 16
    backend_name: str = _BACKEND_NAME


@dataclass(frozen=True)
class PreparedW8A16TiledFusedMoEWeights:
    """Per-output-channel INT8 weights (packed, fp32 scales) against BF16 activations."""

    w13: tuple[torch.Tensor, int, int, torch.Tensor]
    w2: tuple[torch.Tensor, int, int, torch.Tensor]
    fused_silu: bool = True
    gemm_backend: int = _BACKEND_ID
    backend_n_tile: int = 16
    backend_name: str = "gfx950_w8a16_mfma"


@dataclass(frozen=True)
class PreparedW8A8TiledFusedMoEWeights:
    """Per-channel W8 weights (packed int8, fp32 scales) for dynamic-A8 MoE."""

    w13: tuple[torch.Tensor, int, int, torch.Tensor]
    w2: tuple[torch.Tensor, int, int, torch.Tensor]
    fused_silu: bool = True
    gemm_backend: int = _BACKEND_ID
    backend_n_tile: int = 16
    backend_name: str = "gfx950_w8a8_mfma"


@dataclass(frozen=True)
class PreparedBF16TiledRoutedSharedMoEWeights:
    """One routed expert array followed by one synthetic shared expert."""

    packed: PreparedBF16TiledFusedMoEWeights
    routed_experts: int
    shared_expert_id: int


@dataclass(frozen=True)
class PreparedW8A16TiledRoutedSharedMoEWeights:
    packed: PreparedW8A16TiledFusedMoEWeights
    routed_experts: int
    shared_expert_id: int


@dataclass(frozen=True)
class PreparedW8A8TiledRoutedSharedMoEWeights:
    """Dynamic-A8 routed experts followed by one synthetic shared expert."""

    packed: PreparedW8A8TiledFusedMoEWeights
    routed_experts: int
    shared_expert_id: int


_HAS_BF16_TILED_FUSED_MOE = _native.moe_C is not None and _native.gpu_available()
_HAS_W8A8_TILED_FUSED_MOE = _HAS_BF16_TILED_FUSED_MOE

_INTEGER_DTYPES = {torch.int8, torch.int16, torch.int32, torch.int64}


def _require_backend() -> None:
    _native.require_native()
    if not _native.gpu_available():
        raise RuntimeError("No BF16 tiled fused MoE backend is supported: no ROCm device is visible")


def available_fused_moe_bf16_tiled_backends() -> tuple[str, ...]:
    """Return native MoE backends usable by the current process."""
    if _native.moe_C is None or not _native.gpu_available():
        return ()
    return tuple(str(name) for name in _native.moe_C.available_backends())


def _activation_name(activation: Any) -> str:
    value = getattr(activation, "value", activation)
    if not isinstance(value, str):
        value = str(value)
    value = {"gelu_pytorch_tanh": "gelu_tanh"}.get(value, value)
    if value not in {"silu", "gelu", "swigluoai"}:
        raise ValueError(f"Unsupported MoE activation {value!r}; supported activations: gelu, silu, swigluoai")
    return value


def _native_activation_name(activation: Any, weights: Any, swiglu_limit: float | None) -> str:
    """bf16_tiled.py:245-260: limit None/0 keeps the activation, 10 selects the clamp."""
    name = _activation_name(activation)
    if swiglu_limit is None or float(swiglu_limit) == 0.0:
        return name
    limit = float(swiglu_limit)
    if not math.isfinite(limit) or limit != 10.0:
        raise ValueError("clamped SwiGLU currently requires swiglu_limit=10.0")
    if name != "silu":
        raise ValueError("swiglu_limit is only valid with activation='silu'")
    if not weights.fused_silu:
        raise ValueError("swiglu_limit requires fused-SiLU weights (prepare with fuse_silu=True)")
    return "silu_clamp10"


def _check_device_tensor(t: torch.Tensor, name: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a ROCm device tensor")


def _validate_output_buffer(input: torch.Tensor, out: torch.Tensor | None) -> None:
    if out is None:
        return
    if tuple(out.shape) != tuple(input.shape):
        raise ValueError(f"out must have shape {tuple(input.shape)}")
    if out.dtype != input.dtype or out.device != input.device:
        raise ValueError("out must match input dtype and device")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    if out.requires_grad:
        raise ValueError("out with requires_grad=True is not supported")


def _check_routing(input: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> None:
    if input.dtype != torch.bfloat16:
        raise TypeError(f"input must be torch.bfloat16, got {input.dtype}")
    _check_device_tensor(input, "input")
    if input.dim() != 2:
        raise ValueError(f"input must be 2-D [tokens, hidden], got {tuple(input.shape)}")
    if topk_ids.dtype not in _INTEGER_DTYPES:
        raise TypeError(f"topk_ids must use an integer dtype, got {topk_ids.dtype}")
    if not topk_weights.dtype.is_floating_point:
        raise TypeError(f"topk_weights must use a floating dtype, got {topk_weights.dtype}")
    if topk_ids.dim() != 2 or topk_weights.dim() != 2 or topk_ids.shape != topk_weights.shape:
        raise ValueError("topk_ids and topk_weights must have matching [tokens, top_k] shapes")
    if int(topk_ids.shape[0]) != int(input.shape[0]) or int(topk_ids.shape[1]) <= 0:
        raise ValueError("topk tensors must match input tokens and have positive top_k")
    if topk_ids.device != input.device or topk_weights.device != input.device:
        raise ValueError("input, topk_ids and topk_weights must share a device")


def _ids(topk_ids: torch.Tensor) -> torch.Tensor:
    if topk_ids.dtype in (torch.int32, torch.int64):
        return topk_ids.contiguous()
    return topk_ids.to(torch.int32).contiguous()


def _weights_f32(topk_weights: torch.Tensor, scaling: float = 1.0) -> tuple[torch.Tensor, float]:
    """fp32 routing weights; a non-fp32 dtype is scaled in its own dtype first,
    as ``topk_weights * scaling`` is in bf16_tiled.py:1011-1012."""
    if topk_weights.dtype == torch.float32:
        return topk_weights.contiguous(), scaling
    scaled = topk_weights * scaling if scaling != 1.0 else topk_weights
    return scaled.to(torch.float32).contiguous(), 1.0


def _routed_range_checked(routed_experts: int, call):
    """Run a routed+shared forward. The route kernel counts ids outside
    [0, routed_experts) on the device and the extension reads that count once
    after the launch (when id validation is on); an out-of-range id is raised
    as the reference's ValueError (bf16_tiled.py routed+shared wrappers), with
    no host synchronisation before the launch."""
    try:
        return call()
    except RuntimeError as exc:
        if "topk_ids out of range" in str(exc):
            raise ValueError(f"routed topk_ids must be in [0, {routed_experts}): {exc}") from None
        raise


def _to_device(t: torch.Tensor) -> torch.Tensor:
    if t.device.type == "cuda":
        return t.contiguous()
    return t.to(torch.device("cuda", torch.cuda.current_device())).contiguous()


# ---------------------------------------------------------------- prepare --

def prepare_fused_moe_bf16_tiled_weights(
    w13_weight: torch.Tensor,
    w2_weight: torch.Tensor,
    *,
    fuse_silu: bool = False,
    backend: str = "auto",
) -> PreparedBF16TiledFusedMoEWeights:
    """Pack ``[E, 2F, H]`` / ``[E, H, F]`` bf16 expert weights for :func:`fused_moe_bf16_tiled`.

    Replaces bf16_tiled.py:396-450. Any positive H, F are accepted (channel
    groups are padded to 16, K to 64 bytes). ``fuse_silu`` is recorded: the
    GPU W13 epilogue always fuses the activation, the flag only carries the
    reference's call-time checks (clamped SwiGLU requires it).
    """
    _require_backend()
    if w13_weight.dtype != torch.bfloat16 or w2_weight.dtype != torch.bfloat16:
        raise TypeError("BF16 tiled fused MoE weights must be torch.bfloat16")
    if not isinstance(backend, str):
        raise TypeError(f"backend must be a string, got {type(backend).__name__}")
    if backend not in ("auto", _BACKEND_NAME, "arm_sve_bf16", "arm_neon_bf16"):
        raise ValueError(f"unknown MoE backend {backend!r}; available: {_BACKEND_NAME}")
    packed = _native.moe_C.fused_moe_bf16_prepare_weights(_to_device(w13_weight), _to_device(w2_weight))
    return PreparedBF16TiledFusedMoEWeights(
        w13=(packed[0], int(packed[1]), int(packed[2])),
        w2=(packed[3], int(packed[4]), int(packed[5])),
        fused_silu=bool(fuse_silu),
        gemm_backend=int(packed[6]),
        backend_n_tile=int(packed[7]),
        backend_name=str(packed[8]),
    )


def _prepared_w8a8(packed: tuple) -> PreparedW8A8TiledFusedMoEWeights:
    return PreparedW8A8TiledFusedMoEWeights(
        w13=(packed[0], int(packed[1]), int(packed[2]), packed[3]),
        w2=(packed[4], int(packed[5]), int(packed[6]), packed[7]),
        gemm_backend=int(packed[8]),
        backend_n_tile=int(packed[9]),
    )


def prepare_fused_moe_w8a8_tiled_weights(
    w13_weight: torch.Tensor,
    w2_weight: torch.Tensor,
) -> PreparedW8A8TiledFusedMoEWeights:
    """Quantize BF16 expert weights per output channel (on the GPU) for dynamic W8A8.

    scale = max|w|/127 (1 if zero), q = rint(w/scale) clamped to +-127
    (csrc/moe/arm/i8mm_w8a8/kernels.cpp:446-461).
    """
    _require_backend()
    if w13_weight.dtype != torch.bfloat16 or w2_weight.dtype != torch.bfloat16:
        raise TypeError("W8A8 source weights must be torch.bfloat16")
    return _prepared_w8a8(_native.moe_C.fused_moe_w8a8_prepare_weights(_to_device(w13_weight),
                                                                       _to_device(w2_weight)))


def prepare_fused_moe_w8a8_tiled_quantized_weights(
    w13_weight: torch.Tensor,
    w13_scale: torch.Tensor,
    w2_weight: torch.Tensor,
    w2_scale: torch.Tensor,
) -> PreparedW8A8TiledFusedMoEWeights:
    """Pack per-output-channel checkpoint INT8 weights for dynamic W8A8."""
    _require_backend()
    return _prepared_w8a8(_native.moe_C.fused_moe_w8a8_prepare_quantized_weights(
        _to_device(w13_weight), _to_device(w13_scale.float()), _to_device(w2_weight), _to_device(w2_scale.float())))


def prepare_routed_shared_moe_w8a8_tiled_quantized_weights(
    routed_w13_weight: torch.Tensor,
    routed_w13_scale: torch.Tensor,
    routed_w2_weight: torch.Tensor,
    routed_w2_scale: torch.Tensor,
    shared_w13_weight: torch.Tensor,
    shared_w13_scale: torch.Tensor,
    shared_w2_weight: torch.Tensor,
    shared_w2_scale: torch.Tensor,
) -> PreparedW8A8TiledRoutedSharedMoEWeights:
    """Append the shared expert as packed expert E (bf16_tiled.py:573-609)."""
    if shared_w13_weight.dim() != 2 or shared_w2_weight.dim() != 2:
        raise ValueError("shared W8A8 weights must be [2F, H] and [H, F]")
    _require_backend()
    e = int(routed_w13_weight.shape[0])
    # Packed straight into one buffer (no concatenated copy of the sources).
    packed = _prepared_w8a8(_native.moe_C.fused_moe_int8_prepare_routed_shared_weights(
        routed_w13_weight, routed_w13_scale.float(), routed_w2_weight, routed_w2_scale.float(), shared_w13_weight,
        shared_w13_scale.float(), shared_w2_weight, shared_w2_scale.float(), False))
    return PreparedW8A8TiledRoutedSharedMoEWeights(packed=packed, routed_experts=e, shared_expert_id=e)


def prepare_shared_mlp_bf16_tiled_weights(
    w13_weight: torch.Tensor,
    w2_weight: torch.Tensor,
    *,
    backend: str = "auto",
) -> PreparedBF16TiledFusedMoEWeights:
    """Pack one dense gate/up/down MLP ``[2F, H]`` / ``[H, F]`` as a one-expert MoE."""
    if w13_weight.dim() != 2:
        raise ValueError(f"w13_weight must be 2-D [2 * F, H], got shape {tuple(w13_weight.shape)}")
    if w2_weight.dim() != 2:
        raise ValueError(f"w2_weight must be 2-D [H, F], got shape {tuple(w2_weight.shape)}")
    return prepare_fused_moe_bf16_tiled_weights(w13_weight.unsqueeze(0), w2_weight.unsqueeze(0), fuse_silu=True,
                                                backend=backend)


def prepare_routed_shared_moe_bf16_tiled_weights(
    routed_w13_weight: torch.Tensor,
    routed_w2_weight: torch.Tensor,
    shared_w13_weight: torch.Tensor,
    shared_w2_weight: torch.Tensor,
    *,
    backend: str = "auto",
) -> PreparedBF16TiledRoutedSharedMoEWeights:
    """Pack routed experts plus one same-shape shared expert appended as expert E."""
    _require_backend()
    if not isinstance(backend, str):
        raise TypeError(f"backend must be a string, got {type(backend).__name__}")
    if shared_w13_weight.dim() == 3:
        shared_w13_weight = shared_w13_weight.squeeze(0)
    if shared_w2_weight.dim() == 3:
        shared_w2_weight = shared_w2_weight.squeeze(0)
    if backend not in ("auto", _BACKEND_NAME, "arm_sve_bf16", "arm_neon_bf16"):
        raise ValueError(f"unknown MoE backend {backend!r}; available: {_BACKEND_NAME}")
    if any(t.dtype != torch.bfloat16 for t in (routed_w13_weight, routed_w2_weight, shared_w13_weight,
                                                shared_w2_weight)):
        raise TypeError("BF16 tiled fused MoE weights must be torch.bfloat16")
    # Packed straight into one buffer (no concatenated copy of the sources).
    packed = _native.moe_C.fused_moe_bf16_prepare_routed_shared_weights(routed_w13_weight, routed_w2_weight,
                                                                        shared_w13_weight, shared_w2_weight)
    combined = PreparedBF16TiledFusedMoEWeights(
        w13=(packed[0], int(packed[1]), int(packed[2])),
        w2=(packed[3], int(packed[4]), int(packed[5])),
        fused_silu=True,
        gemm_backend=int(packed[6]),
        backend_n_tile=int(packed[7]),
        backend_name=str(packed[8]),
    )
    e = int(routed_w13_weight.shape[0])
    return PreparedBF16TiledRoutedSharedMoEWeights(packed=combined, routed_experts=e, shared_expert_id=e)


def _prepared_w8a16(packed: tuple) -> PreparedW8A16TiledFusedMoEWeights:
    return PreparedW8A16TiledFusedMoEWeights(
        w13=(packed[0], int(packed[1]), int(packed[2]), packed[3]),
        w2=(packed[4], int(packed[5]), int(packed[6]), packed[7]),
        gemm_backend=int(packed[8]),
        backend_n_tile=int(packed[9]),
    )


def prepare_fused_moe_w8a16_tiled_weights(
    w13_weight: torch.Tensor,
    w2_weight: torch.Tensor,
) -> PreparedW8A16TiledFusedMoEWeights:
    """Quantize BF16 expert weights to symmetric per-output-channel INT8 (bf16_tiled.py:453-472).

    scale = max|w|/127 (1 if zero), q = nearbyint(w/scale) clamped to +-127
    (fused_moe_bf16_tiled.cpp:4947-4976), computed on the GPU. The packed layout
    is the W8A8 one: the weights stream through the same MFMA operand tiles.
    """
    _require_backend()
    if w13_weight.dtype != torch.bfloat16 or w2_weight.dtype != torch.bfloat16:
        raise TypeError("W8A16 source weights must be torch.bfloat16")
    return _prepared_w8a16(_native.moe_C.fused_moe_w8a16_prepare_weights(_to_device(w13_weight),
                                                                         _to_device(w2_weight)))


def prepare_fused_moe_w8a16_tiled_quantized_weights(
    w13_weight: torch.Tensor,
    w13_scale: torch.Tensor,
    w2_weight: torch.Tensor,
    w2_scale: torch.Tensor,
) -> PreparedW8A16TiledFusedMoEWeights:
    """Pack checkpoint INT8 expert weights without dequantizing or requantizing (bf16_tiled.py:484-499)."""
    _require_backend()
    return _prepared_w8a16(_native.moe_C.fused_moe_w8a16_prepare_quantized_weights(
        _to_device(w13_weight), _to_device(w13_scale.float()), _to_device(w2_weight), _to_device(w2_scale.float())))


def prepare_routed_shared_moe_w8a16_tiled_quantized_weights(
    routed_w13_weight: torch.Tensor,
    routed_w13_scale: torch.Tensor,
    routed_w2_weight: torch.Tensor,
    routed_w2_scale: torch.Tensor,
    shared_w13_weight: torch.Tensor,
    shared_w13_scale: torch.Tensor,
    shared_w2_weight: torch.Tensor,
    shared_w2_scale: torch.Tensor,
) -> PreparedW8A16TiledRoutedSharedMoEWeights:
    """Routed checkpoint INT8 experts plus one same-shape shared expert appended as expert E
    (bf16_tiled.py:541-570; native fused_moe_bf16_tiled.cpp:6276-6288)."""
    if shared_w13_weight.dim() != 2 or shared_w2_weight.dim() != 2:
        raise ValueError("shared W8A16 weights must be [2F, H] and [H, F]")
    _require_backend()
    e = int(routed_w13_weight.shape[0])
    # Packed straight into one buffer (no concatenated copy of the sources).
    packed = _prepared_w8a16(_native.moe_C.fused_moe_int8_prepare_routed_shared_weights(
        routed_w13_weight, routed_w13_scale.float(), routed_w2_weight, routed_w2_scale.float(), shared_w13_weight,
        shared_w13_scale.float(), shared_w2_weight, shared_w2_scale.float(), True))
    return PreparedW8A16TiledRoutedSharedMoEWeights(packed=packed, routed_experts=e, shared_expert_id=e)


# ---------------------------------------------------------------- BF16 ops --

def _bf16_call(input, weights, topk_weights, topk_ids, *, w13_bias, w2_bias, activation, global_num_experts,
               skip_weighted, shared_id, scaling, out):
    w13, w2 = weights.w13, weights.w2
    return _native.moe_C.fused_moe_bf16_forward(
        input.contiguous(), w13[0], int(w13[1]), int(w13[2]), w2[0], int(w2[1]), int(w2[2]), topk_weights, topk_ids,
        w13_bias, w2_bias, activation, int(global_num_experts), bool(skip_weighted), int(shared_id), float(scaling),
        out, _native.validate_ids_default())


def fused_moe_bf16_tiled(
    input: torch.Tensor,
    weights: PreparedBF16TiledFusedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    *,
    w13_bias: torch.Tensor | None = None,
    w2_bias: torch.Tensor | None = None,
    num_threads: int = 1,
    activation: Any = "silu",
    global_num_experts: int = -1,
    skip_weighted: bool = False,
    silu_poly_degree: int = 5,
    swiglu_limit: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """BF16 fused MoE (bf16_tiled.py:676-775) on bf16 MFMA with fp32 accumulation.

    ``silu_poly_degree`` is accepted for compatibility (4/5/6); ``num_threads``
    must be positive and is otherwise unused. A supplied ``out`` is written in
    place and returned.
    """
    _require_backend()
    _check_routing(input, topk_weights, topk_ids)
    if int(num_threads) <= 0:
        raise ValueError(f"num_threads must be positive, got {num_threads}")
    if int(silu_poly_degree) not in (4, 5, 6):
        raise ValueError("silu_poly_degree must be 4, 5 or 6")
    if bool(skip_weighted) and int(topk_ids.shape[1]) != 1:
        raise ValueError("skip_weighted is only valid when top_k == 1")
    experts = int(weights.w13[0].shape[0])
    if global_num_experts != -1 and not (0 < int(global_num_experts) <= experts):
        raise RuntimeError(f"global_num_experts must be positive and <= {experts}, got {global_num_experts}")
    native_act = _native_activation_name(activation, weights, swiglu_limit)
    if weights.fused_silu and native_act not in ("silu", "silu_clamp10"):
        raise RuntimeError("fused-SiLU weights require activation='silu'")
    _validate_output_buffer(input, out)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w, _ = _weights_f32(topk_weights)
    return _bf16_call(input, weights, w, _ids(topk_ids), w13_bias=w13_bias, w2_bias=w2_bias, activation=native_act,
                      global_num_experts=global_num_experts, skip_weighted=skip_weighted, shared_id=-1,
                      scaling=1.0, out=out)


def fused_moe_bf16_tiled_with_shared(
    input: torch.Tensor,
    weights: PreparedBF16TiledRoutedSharedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    *,
    num_threads: int = 1,
    routed_scaling_factor: float = 1.0,
    activation: Any = "silu",
    silu_poly_degree: int = 5,
    swiglu_limit: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Routed experts plus one all-token shared expert (bf16_tiled.py:778-878).

    The shared expert is slot k of every token with weight 1.0; routed weights
    are multiplied by ``routed_scaling_factor``. The appended slot is built on
    the GPU inside the route kernel instead of a host-side concatenation.
    """
    _require_backend()
    if not isinstance(weights, PreparedBF16TiledRoutedSharedMoEWeights):
        raise TypeError("weights must be PreparedBF16TiledRoutedSharedMoEWeights")
    _check_routing(input, topk_weights, topk_ids)
    if int(num_threads) <= 0:
        raise ValueError(f"num_threads must be positive, got {num_threads}")
    scaling = float(routed_scaling_factor)
    if not math.isfinite(scaling):
        raise ValueError("routed_scaling_factor must be finite")
    native_act = _native_activation_name(activation, weights.packed, swiglu_limit)
    if _activation_name(activation) != "silu":
        raise ValueError("routed+shared BF16 scheduling currently requires activation='silu'")
    _validate_output_buffer(input, out)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w, scale = _weights_f32(topk_weights, scaling)
    return _routed_range_checked(weights.routed_experts, lambda: _bf16_call(
        input, weights.packed, w, _ids(topk_ids), w13_bias=None, w2_bias=None, activation=native_act,
        global_num_experts=weights.routed_experts, skip_weighted=False, shared_id=weights.shared_expert_id,
        scaling=scale, out=out))


def shared_mlp_bf16_tiled(
    input: torch.Tensor,
    weights: PreparedBF16TiledFusedMoEWeights,
    *,
    thread_cpu_ids: torch.Tensor | None = None,
    num_threads: int = 1,
    silu_poly_degree: int = 5,
    swiglu_limit: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One packed expert as a dense shared MLP (bf16_tiled.py:1805-1873).

    Runs the MoE pipeline with every token routed to expert 0 with weight 1,
    which writes the same bf16 values as a direct W2 store.
    """
    _require_backend()
    if input.dtype != torch.bfloat16:
        raise TypeError(f"input must be torch.bfloat16, got {input.dtype}")
    _check_device_tensor(input, "input")
    if int(num_threads) <= 0:
        raise ValueError(f"num_threads must be positive, got {num_threads}")
    if not weights.fused_silu:
        raise ValueError("shared MLP requires weights prepared with fuse_silu=True")
    if int(weights.w13[0].size(0)) != 1 or int(weights.w2[0].size(0)) != 1:
        raise ValueError("shared MLP requires exactly one packed expert")
    if thread_cpu_ids is not None and int(thread_cpu_ids.numel()) != int(num_threads):
        raise ValueError(
            f"thread_cpu_ids must have exactly num_threads entries: got {int(thread_cpu_ids.numel())} vs {int(num_threads)}")
    _validate_output_buffer(input, out)
    native_act = _native_activation_name("silu", weights, swiglu_limit)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w13, w2 = weights.w13, weights.w2
    return _native.moe_C.fused_moe_bf16_forward(
        input.contiguous(), w13[0], int(w13[1]), int(w13[2]), w2[0], int(w2[1]), int(w2[2]), None, None, None, None,
        native_act, -1, False, 0, 1.0, out, False)


def _delegate_bf16(input, weights, topk_weights, topk_ids, *, global_num_experts=-1, silu_poly_degree=5,
                   out=None, **kwargs):
    return fused_moe_bf16_tiled(input, weights, topk_weights, topk_ids, global_num_experts=global_num_experts,
                                silu_poly_degree=silu_poly_degree, out=out, **kwargs)


def fused_moe_bf16_tiled_scheduled(input, weights, topk_weights, topk_ids, wave_offsets, team_expert_ids,
                                   team_threads, *, thread_cpu_ids=None, w13_bias=None, w2_bias=None,
                                   num_threads: int = 1, activation: Any = "silu", global_num_experts: int = -1,
                                   skip_weighted: bool = False, silu_poly_degree: int = 5, out=None):
    """CPU team schedules select nothing on the GPU: runs :func:`fused_moe_bf16_tiled`."""
    return fused_moe_bf16_tiled(input, weights, topk_weights, topk_ids, w13_bias=w13_bias, w2_bias=w2_bias,
                                num_threads=num_threads, activation=activation,
                                global_num_experts=global_num_experts, skip_weighted=skip_weighted,
                                silu_poly_degree=silu_poly_degree, out=out)


def fused_moe_bf16_tiled_async(input, weights, topk_weights, topk_ids, task_expert_ids, task_core_begins,
                               task_threads, task_dep_offsets, task_deps, *, thread_cpu_ids=None, w13_bias=None,
                               w2_bias=None, num_threads: int = 1, activation: Any = "silu",
                               global_num_experts: int = -1, skip_weighted: bool = False,
                               silu_poly_degree: int = 5, out=None):
    """CPU async task graphs select nothing on the GPU: runs :func:`fused_moe_bf16_tiled`."""
    return fused_moe_bf16_tiled(input, weights, topk_weights, topk_ids, w13_bias=w13_bias, w2_bias=w2_bias,
                                num_threads=num_threads, activation=activation,
                                global_num_experts=global_num_experts, skip_weighted=skip_weighted,
                                silu_poly_degree=silu_poly_degree, out=out)


def fused_moe_bf16_tiled_async_plan(input, weights, topk_weights, topk_ids, plan, *, w13_bias=None, w2_bias=None,
                                    activation: Any = "silu", global_num_experts: int = -1,
                                    skip_weighted: bool = False, silu_poly_degree: int = 5,
                                    swiglu_limit: float | None = None, out=None):
    """Validates the Plan V2 schema, then runs :func:`fused_moe_bf16_tiled`."""
    materialize_plan(plan)
    return fused_moe_bf16_tiled(input, weights, topk_weights, topk_ids, w13_bias=w13_bias, w2_bias=w2_bias,
                                activation=activation, global_num_experts=global_num_experts,
                                skip_weighted=skip_weighted, silu_poly_degree=silu_poly_degree,
                                swiglu_limit=swiglu_limit, out=out)


def fused_moe_bf16_tiled_planned_staged(input, weights, topk_weights, topk_ids, w13_plan, w2_plan, *,
                                        global_num_experts: int = -1, silu_poly_degree: int = 5, out=None):
    """Validates both plans, then runs :func:`fused_moe_bf16_tiled` (W13 and W2 are separate launches anyway)."""
    materialize_plan(w13_plan)
    materialize_plan(w2_plan)
    if not weights.fused_silu:
        raise ValueError("planned-staged MoE requires weights prepared with fuse_silu=True")
    return fused_moe_bf16_tiled(input, weights, topk_weights, topk_ids, global_num_experts=global_num_experts,
                                silu_poly_degree=silu_poly_degree, out=out)


def fused_moe_bf16_tiled_vllm_staged(input, weights, topk_weights, topk_ids, *, thread_cpu_ids=None,
                                     num_threads: int = 1, global_num_experts: int = -1,
                                     silu_poly_degree: int = 5, out=None):
    """The staged W13-then-W2 order is this backend's only order: runs :func:`fused_moe_bf16_tiled`."""
    if not weights.fused_silu:
        raise ValueError("vLLM-staged baseline requires weights prepared with fuse_silu=True")
    if thread_cpu_ids is not None and int(thread_cpu_ids.numel()) != int(num_threads):
        raise ValueError("thread_cpu_ids must have exactly num_threads entries")
    return fused_moe_bf16_tiled(input, weights, topk_weights, topk_ids, num_threads=num_threads,
                                global_num_experts=global_num_experts, silu_poly_degree=silu_poly_degree, out=out)


# ---------------------------------------------------------------- W8A8 ops --

def _w8a8_call(input, weights, topk_weights, topk_ids, *, shared_id, scaling, out, valid_experts=-1):
    w13, w2 = weights.w13, weights.w2
    return _native.moe_C.fused_moe_w8a8_forward(
        input.contiguous(), w13[0], int(w13[1]), int(w13[2]), w13[3], w2[0], int(w2[1]), int(w2[2]), w2[3],
        topk_weights, topk_ids, int(shared_id), float(scaling), int(valid_experts), out,
        _native.validate_ids_default())


def _check_w8a8_call(input, weights, topk_weights, topk_ids, activation, swiglu_limit, global_num_experts,
                     skip_weighted, out):
    if not isinstance(weights, PreparedW8A8TiledFusedMoEWeights):
        raise TypeError("weights must be PreparedW8A8TiledFusedMoEWeights")
    if input.dtype != torch.bfloat16:
        raise TypeError("W8A8 input must be a torch.bfloat16 tensor")
    if _activation_name(activation) != "silu" or float(swiglu_limit) != 10.0:
        raise ValueError("W8A8 supports only activation='silu' with swiglu_limit=10.0")
    _check_routing(input, topk_weights, topk_ids)
    if int(global_num_experts) != -1:
        raise RuntimeError("W8A8 does not support expert-parallel id remapping (global_num_experts must be -1)")
    if bool(skip_weighted):
        raise RuntimeError("W8A8 requires weighted TopK merge")
    _validate_output_buffer(input, out)


def fused_moe_w8a8_tiled_async_plan(
    input: torch.Tensor,
    weights: PreparedW8A8TiledFusedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    plan: AsyncMoEPlanV2 | Mapping[str, object],
    *,
    activation: Any = "silu",
    global_num_experts: int = -1,
    skip_weighted: bool = False,
    swiglu_limit: float = 10.0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dynamic-per-row W8A8 experts (bf16_tiled.py:1450-1523); the plan is schema-checked only."""
    _require_backend()
    _check_w8a8_call(input, weights, topk_weights, topk_ids, activation, swiglu_limit, global_num_experts,
                     skip_weighted, out)
    materialize_plan(plan)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w, _ = _weights_f32(topk_weights)
    return _w8a8_call(input, weights, w, _ids(topk_ids), shared_id=-1, scaling=1.0, out=out)


def fused_moe_w8a8_tiled(
    input: torch.Tensor,
    weights: PreparedW8A8TiledFusedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    *,
    num_threads: int = 1,
    activation: Any = "silu",
    global_num_experts: int = -1,
    skip_weighted: bool = False,
    swiglu_limit: float = 10.0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """W8A8 MoE (bf16_tiled.py:1526-1573). No planner runtime is required on the GPU."""
    _require_backend()
    if not isinstance(weights, PreparedW8A8TiledFusedMoEWeights):
        raise TypeError("weights must be PreparedW8A8TiledFusedMoEWeights")
    if int(num_threads) <= 0:
        raise ValueError(f"num_threads must be positive, got {num_threads}")
    _check_w8a8_call(input, weights, topk_weights, topk_ids, activation, swiglu_limit, global_num_experts,
                     skip_weighted, out)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w, _ = _weights_f32(topk_weights)
    return _w8a8_call(input, weights, w, _ids(topk_ids), shared_id=-1, scaling=1.0, out=out)


def fused_moe_w8a8_tiled_with_shared(
    input: torch.Tensor,
    weights: PreparedW8A8TiledRoutedSharedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    *,
    num_threads: int = 1,
    routed_scaling_factor: float = 1.0,
    activation: Any = "silu",
    swiglu_limit: float = 10.0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dynamic W8A8 routed experts plus one all-token shared expert (bf16_tiled.py:964-1040)."""
    _require_backend()
    if not isinstance(weights, PreparedW8A8TiledRoutedSharedMoEWeights):
        raise TypeError("weights must be PreparedW8A8TiledRoutedSharedMoEWeights")
    if input.dtype != torch.bfloat16:
        raise TypeError("input must be a torch.bfloat16 tensor")
    _check_routing(input, topk_weights, topk_ids)
    if int(num_threads) <= 0:
        raise ValueError(f"num_threads must be positive, got {num_threads}")
    scaling = float(routed_scaling_factor)
    if not math.isfinite(scaling):
        raise ValueError("routed_scaling_factor must be finite")
    if _activation_name(activation) != "silu" or float(swiglu_limit) != 10.0:
        raise ValueError("routed+shared W8A8 requires activation='silu' with swiglu_limit=10.0")
    _validate_output_buffer(input, out)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w, scale = _weights_f32(topk_weights, scaling)
    return _routed_range_checked(weights.routed_experts, lambda: _w8a8_call(
        input, weights.packed, w, _ids(topk_ids), shared_id=weights.shared_expert_id, scaling=scale, out=out,
        valid_experts=weights.routed_experts))


# --------------------------------------------------------------- W8A16 ops --

def _w8a16_call(input, weights, topk_weights, topk_ids, *, activation, global_num_experts, skip_weighted, shared_id,
                scaling, out):
    w13, w2 = weights.w13, weights.w2
    return _native.moe_C.fused_moe_w8a16_forward(
        input.contiguous(), w13[0], int(w13[1]), int(w13[2]), w13[3], w2[0], int(w2[1]), int(w2[2]), w2[3],
        topk_weights, topk_ids, activation, int(global_num_experts), bool(skip_weighted), int(shared_id),
        float(scaling), out, _native.validate_ids_default())


def _w8a16_activation(activation: Any, weights: PreparedW8A16TiledFusedMoEWeights, swiglu_limit) -> str:
    native = _native_activation_name(activation, weights, swiglu_limit)
    if native not in ("silu", "silu_clamp10", "gelu"):
        raise ValueError(f"W8A16 fused MoE supports silu (optionally clamped) and gelu, got {native!r}")
    return native


def _check_w8a16_call(input, weights, topk_weights, topk_ids, num_threads, global_num_experts, skip_weighted,
                      silu_poly_degree, out):
    if not isinstance(weights, PreparedW8A16TiledFusedMoEWeights):
        raise TypeError("weights must be PreparedW8A16TiledFusedMoEWeights")
    if input.dtype != torch.bfloat16:
        raise TypeError("W8A16 input must be a torch.bfloat16 tensor")
    if topk_ids.dtype not in _INTEGER_DTYPES:
        raise TypeError(f"topk_ids must use an integer dtype, got {topk_ids.dtype}")
    if not topk_weights.dtype.is_floating_point:
        raise TypeError(f"topk_weights must use a floating dtype, got {topk_weights.dtype}")
    _check_routing(input, topk_weights, topk_ids)
    if int(num_threads) <= 0:
        raise ValueError(f"num_threads must be positive, got {num_threads}")
    if int(silu_poly_degree) not in (4, 5, 6):
        raise ValueError("silu_poly_degree must be 4, 5 or 6")
    if bool(skip_weighted) and int(topk_ids.shape[1]) != 1:
        raise ValueError("skip_weighted is only valid when top_k == 1")
    experts = int(weights.w13[0].shape[0])
    if global_num_experts != -1 and not (0 < int(global_num_experts) <= experts):
        raise RuntimeError(f"global_num_experts must be positive and <= {experts}, got {global_num_experts}")
    _validate_output_buffer(input, out)


def fused_moe_w8a16_tiled_async_plan(
    input: torch.Tensor,
    weights: PreparedW8A16TiledFusedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    plan: AsyncMoEPlanV2 | Mapping[str, object],
    *,
    activation: Any = "silu",
    global_num_experts: int = -1,
    skip_weighted: bool = False,
    silu_poly_degree: int = 5,
    swiglu_limit: float | None = None,
    cache_dequant: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-channel W8A16 experts (bf16_tiled.py:1309-1373); the plan is schema-checked only."""
    _require_backend()
    materialize_plan(plan)
    return fused_moe_w8a16_tiled(input, weights, topk_weights, topk_ids, activation=activation,
                                 global_num_experts=global_num_experts, skip_weighted=skip_weighted,
                                 silu_poly_degree=silu_poly_degree, swiglu_limit=swiglu_limit,
                                 cache_dequant=cache_dequant, out=out)


def fused_moe_w8a16_tiled(
    input: torch.Tensor,
    weights: PreparedW8A16TiledFusedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    *,
    num_threads: int = 1,
    activation: Any = "silu",
    global_num_experts: int = -1,
    skip_weighted: bool = False,
    silu_poly_degree: int = 5,
    swiglu_limit: float | None = None,
    cache_dequant: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """W8A16 fused MoE (bf16_tiled.py:1376-1447) on bf16 MFMA.

    INT8 weights are widened to bf16 in registers (exact) and accumulate against
    the bf16 activations in fp32; each output channel's scale multiplies its
    accumulator. ``cache_dequant`` selects a CPU dequantised-window cache in the
    reference and changes nothing here (weights are never dequantised to memory).
    No planner runtime is required on the GPU.
    """
    _require_backend()
    _check_w8a16_call(input, weights, topk_weights, topk_ids, num_threads, global_num_experts, skip_weighted,
                      silu_poly_degree, out)
    native_act = _w8a16_activation(activation, weights, swiglu_limit)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w, _ = _weights_f32(topk_weights)
    return _w8a16_call(input, weights, w, _ids(topk_ids), activation=native_act,
                       global_num_experts=global_num_experts, skip_weighted=skip_weighted, shared_id=-1, scaling=1.0,
                       out=out)


def fused_moe_w8a16_tiled_with_shared(
    input: torch.Tensor,
    weights: PreparedW8A16TiledRoutedSharedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    *,
    num_threads: int = 1,
    routed_scaling_factor: float = 1.0,
    activation: Any = "silu",
    silu_poly_degree: int = 5,
    swiglu_limit: float | None = None,
    cache_dequant: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Checkpoint W8A16 routed experts with one all-token shared expert (bf16_tiled.py:881-961).

    The shared expert is slot k of every token with weight 1.0; routed weights
    are multiplied by ``routed_scaling_factor`` inside the route kernel.
    """
    _require_backend()
    if not isinstance(weights, PreparedW8A16TiledRoutedSharedMoEWeights):
        raise TypeError("weights must be PreparedW8A16TiledRoutedSharedMoEWeights")
    if input.dtype != torch.bfloat16:
        raise TypeError("input must be a torch.bfloat16 tensor")
    _check_routing(input, topk_weights, topk_ids)
    if int(topk_ids.shape[1]) <= 0:
        raise ValueError("topk tensors must match input tokens and have positive top_k")
    if int(num_threads) <= 0:
        raise ValueError(f"num_threads must be positive, got {num_threads}")
    scaling = float(routed_scaling_factor)
    if not math.isfinite(scaling):
        raise ValueError("routed_scaling_factor must be finite")
    native_act = _w8a16_activation(activation, weights.packed, swiglu_limit)
    if _activation_name(activation) != "silu":
        raise ValueError("routed+shared W8A16 scheduling currently requires activation='silu'")
    _validate_output_buffer(input, out)
    if int(input.shape[0]) == 0:
        return out if out is not None else torch.empty_like(input)
    w, scale = _weights_f32(topk_weights, scaling)
    return _routed_range_checked(weights.routed_experts, lambda: _w8a16_call(
        input, weights.packed, w, _ids(topk_ids), activation=native_act, global_num_experts=weights.routed_experts,
        skip_weighted=False, shared_id=weights.shared_expert_id, scaling=scale, out=out))


# ------------------------------------------------------------- dispatcher --

def fused_moe_tiled(
    input: torch.Tensor,
    weights: PreparedBF16TiledFusedMoEWeights | PreparedW8A16TiledFusedMoEWeights | PreparedW8A8TiledFusedMoEWeights,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    *,
    w13_bias: torch.Tensor | None = None,
    w2_bias: torch.Tensor | None = None,
    num_threads: int = 1,
    activation: Any = "silu",
    global_num_experts: int = -1,
    skip_weighted: bool = False,
    silu_poly_degree: int = 5,
    swiglu_limit: float | None = None,
    cache_dequant: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dispatch on the prepared-weight type (bf16_tiled.py:1576-1642)."""
    common = {
        "num_threads": num_threads,
        "activation": activation,
        "global_num_experts": global_num_experts,
        "skip_weighted": skip_weighted,
        "silu_poly_degree": silu_poly_degree,
        "swiglu_limit": swiglu_limit,
        "out": out,
    }
    if isinstance(weights, PreparedBF16TiledFusedMoEWeights):
        if cache_dequant:
            raise ValueError("cache_dequant is supported only by W8A16 fused MoE weights")
        return fused_moe_bf16_tiled(input, weights, topk_weights, topk_ids, w13_bias=w13_bias, w2_bias=w2_bias,
                                    **common)
    if isinstance(weights, PreparedW8A16TiledFusedMoEWeights):
        if w13_bias is not None or w2_bias is not None:
            raise ValueError("W8A16 fused MoE does not support w13_bias or w2_bias")
        return fused_moe_w8a16_tiled(input, weights, topk_weights, topk_ids, cache_dequant=cache_dequant, **common)
    if isinstance(weights, PreparedW8A8TiledFusedMoEWeights):
        if w13_bias is not None or w2_bias is not None:
            raise ValueError("W8A8 fused MoE does not support w13_bias or w2_bias")
        if cache_dequant:
            raise ValueError("cache_dequant is supported only by W8A16 fused MoE weights")
        common.pop("silu_poly_degree")
        if common["swiglu_limit"] is None:
            common["swiglu_limit"] = 10.0
        return fused_moe_w8a8_tiled(input, weights, topk_weights, topk_ids, **common)
    raise TypeError(
        "weights must be PreparedBF16TiledFusedMoEWeights, "
        "PreparedW8A16TiledFusedMoEWeights, or PreparedW8A8TiledFusedMoEWeights"
    )


bf16_tiled_fused_moe = fused_moe_bf16_tiled
bf16_tiled_fused_moe_scheduled = fused_moe_bf16_tiled_scheduled
bf16_tiled_fused_moe_async = fused_moe_bf16_tiled_async
bf16_tiled_fused_moe_async_plan = fused_moe_bf16_tiled_async_plan
bf16_tiled_fused_moe_planned_staged = fused_moe_bf16_tiled_planned_staged
bf16_tiled_fused_moe_vllm_staged = fused_moe_bf16_tiled_vllm_staged
prepare_bf16_tiled_fused_moe_weights = prepare_fused_moe_bf16_tiled_weights

__all__ = [
    "PreparedBF16TiledFusedMoEWeights",
    "PreparedBF16TiledRoutedSharedMoEWeights",
    "PreparedW8A16TiledFusedMoEWeights",
    "PreparedW8A8TiledFusedMoEWeights",
    "PreparedW8A16TiledRoutedSharedMoEWeights",
    "PreparedW8A8TiledRoutedSharedMoEWeights",
    "PreparedWeight",
    "_HAS_BF16_TILED_FUSED_MOE",
    "_HAS_W8A8_TILED_FUSED_MOE",
    "available_fused_moe_bf16_tiled_backends",
    "fused_moe_bf16_tiled",
    "fused_moe_bf16_tiled_with_shared",
    "fused_moe_bf16_tiled_scheduled",
    "fused_moe_bf16_tiled_async",
    "fused_moe_bf16_tiled_async_plan",
    "fused_moe_bf16_tiled_planned_staged",
    "fused_moe_bf16_tiled_vllm_staged",
    "fused_moe_tiled",
    "fused_moe_w8a16_tiled",
    "fused_moe_w8a16_tiled_async_plan",
    "fused_moe_w8a8_tiled",
    "fused_moe_w8a8_tiled_async_plan",
    "fused_moe_w8a16_tiled_with_shared",
    "fused_moe_w8a8_tiled_with_shared",
    "shared_mlp_bf16_tiled",
    "bf16_tiled_fused_moe",
    "bf16_tiled_fused_moe_scheduled",
    "bf16_tiled_fused_moe_async",
    "bf16_tiled_fused_moe_async_plan",
    "bf16_tiled_fused_moe_planned_staged",
    "bf16_tiled_fused_moe_vllm_staged",
    "prepare_fused_moe_bf16_tiled_weights",
    "prepare_fused_moe_w8a16_tiled_weights",
    "prepare_fused_moe_w8a16_tiled_quantized_weights",
    "prepare_fused_moe_w8a8_tiled_weights",
    "prepare_fused_moe_w8a8_tiled_quantized_weights",
    "prepare_routed_shared_moe_bf16_tiled_weights",
    "prepare_routed_shared_moe_w8a16_tiled_quantized_weights",
    "prepare_routed_shared_moe_w8a8_tiled_quantized_weights",
    "prepare_shared_mlp_bf16_tiled_weights",
    "prepare_bf16_tiled_fused_moe_weights",
]
