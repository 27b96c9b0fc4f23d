"""fused_cpp_amd -- MI355X (gfx950) fused MoE operators.

Drop-in for the fused-MoE path of hearth-stone/fused_cpp: ``moe`` mirrors
``fused_cpp.moe`` and ``i8gemm`` mirrors ``fused_cpp.i8gemm``. The operators
run hand-written HIP kernels (libfcmoe.so, C ABI in include/fcmoe.h) through
the C++ torch extension ``_moe_C``. ``deepseek_v4_w8a8`` mirrors
``fused_cpp.deepseek_v4_w8a8`` (W8A8 attention linears on i8gemm); ``router``
adds the caller-side top-k softmax router as a GPU kernel.
"""

from . import deepseek_v4_w8a8, i8gemm, moe, router

__all__ = ["deepseek_v4_w8a8", "i8gemm", "moe", "router"]
