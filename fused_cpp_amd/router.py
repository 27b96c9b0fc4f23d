"""Top-k softmax router on MI355X: the caller step that produces the
``topk_ids`` / ``topk_weights`` the fused-MoE ops consume.

The reference receives these from its caller (src/fused_cpp/moe/bf16_tiled.py:676-681;
the vLLM adapter computes softmax -> top-k -> renormalise -> routed scaling,
docs/vllm_bf16_tiled_moe_integration.md:75-87). ``topk_softmax`` runs that step
as one HIP kernel (``fcmoe_router_topk``), so a MoE layer needs no host round trip.
"""

from __future__ import annotations

import ctypes

import torch

from fused_cpp_amd import cabi


def topk_softmax(logits: torch.Tensor, top_k: int, *, renormalize: bool = True, scale: float = 1.0,
                 ids_dtype: torch.dtype = torch.int64) -> tuple[torch.Tensor, torch.Tensor]:
    """``logits [T, E]`` fp32 on the ROCm device -> ``(topk_ids [T, k], topk_weights [T, k] fp32)``.

    Ids are in descending logit order (the lower expert id first on equal
    logits). Weights are the softmax probabilities of the selected experts,
    divided by their sum when ``renormalize``, times ``scale``.
    """
    if logits.dim() != 2:
        raise ValueError(f"logits must be 2D [tokens, experts], got {logits.dim()}D")
    if logits.dtype != torch.float32:
        raise TypeError(f"logits must be float32, got {logits.dtype}")
    if logits.device.type != "cuda":
        raise ValueError("logits must be on the ROCm device")
    if ids_dtype not in (torch.int64, torch.int32):
        raise TypeError("ids_dtype must be torch.int64 or torch.int32")
    T, E = logits.shape
    if not 0 < top_k <= min(E, 64) or E > 1024:
        raise ValueError(f"need 0 < top_k <= min(experts, 64) and experts <= 1024 (top_k={top_k}, experts={E})")
    logits = logits.contiguous()
    ids = torch.empty((T, top_k), dtype=ids_dtype, device=logits.device)
    weights = torch.empty((T, top_k), dtype=torch.float32, device=logits.device)
    rc = cabi.lib().fcmoe_router_topk(logits.data_ptr(), T, E, top_k, 1 if renormalize else 0, ctypes.c_float(scale),
                                      ids.data_ptr(), 1 if ids_dtype == torch.int64 else 0, weights.data_ptr(),
                                      cabi.stream_handle())
    cabi.check(rc, "router_topk")
    return ids, weights


__all__ = ["topk_softmax"]
