"""ctypes binding of libfcmoe.so's C ABI (include/fcmoe.h).

This is the binding a non-torch host (or a reference-side FFI) would use; the
GPU parity tests call the kernels through it so that what is checked is the
C ABI itself. Tensors are passed as device pointers (``tensor.data_ptr()``)
with the current torch HIP stream.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

# FCMOE_LIB_DIR: a diagnostic build's directory (python -m fused_cpp_amd.build
# --diag N --out DIR), loaded together with LD_LIBRARY_PATH=DIR so that the
# torch extension resolves the same library
LIB_PATH = Path(os.environ.get("FCMOE_LIB_DIR") or Path(__file__).resolve().parent) / "libfcmoe.so"

FCMOE_ACT_SILU = 0
FCMOE_ACT_GELU = 1
FCMOE_ACT_SWIGLUOAI = 2
FCMOE_ACT_SILU_CLAMP10 = 3

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_SZ = ctypes.c_size_t


class MoeArgs(ctypes.Structure):
    """Mirror of ``struct fcmoe_moe_args``."""

    _fields_ = [
        ("x", _P),
        ("tokens", _I64),
        ("hidden", _I64),
        ("inter", _I64),
        ("topk_ids", _P),
        ("ids_is_i64", _I),
        ("topk_weights", _P),
        ("top_k", _I64),
        ("experts", _I64),
        ("valid_experts", _I64),
        ("shared_expert_id", _I64),
        ("routed_scaling", ctypes.c_float),
        ("w13", _P),
        ("w2", _P),
        ("w13_scale", _P),
        ("w2_scale", _P),
        ("w13_bias", _P),
        ("w2_bias", _P),
        ("activation", _I),
        ("skip_weighted", _I),
        ("out", _P),
        ("invalid_count", _P),
        ("workspace", _P),
        ("workspace_bytes", _SZ),
    ]


# name -> (restype, argtypes); every symbol declared in include/fcmoe.h.
SIGNATURES = {
    "fcmoe_last_error": (ctypes.c_char_p, []),
    "fcmoe_abi_version": (_I, []),
    "fcmoe_quantize_weight_rows": (_I, [_P, _I64, _I64, _P, _P, _P]),
    "fcmoe_packed_expert_bytes": (_I64, [_I, _I64, _I64, _I]),
    "fcmoe_pack_experts": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _P]),
    "fcmoe_route_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "fcmoe_route_build": (_I, [_P, _I, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _SZ, _P]),
    "fcmoe_quantize_rows": (_I, [_P, _I, _I64, _I64, _I, _P, _I64, _P, _P]),
    "fcmoe_router_topk": (_I, [_P, _I64, _I64, _I64, _I, ctypes.c_float, _P, _I, _P, _P]),
    "fcmoe_w8a8_workspace_bytes": (_SZ, [ctypes.POINTER(MoeArgs)]),
    "fcmoe_w8a8_forward": (_I, [ctypes.POINTER(MoeArgs), _P]),
    "fcmoe_w8a8_forward_noalloc": (_I, [ctypes.POINTER(MoeArgs), _P]),
    "fcmoe_bf16_workspace_bytes": (_SZ, [ctypes.POINTER(MoeArgs)]),
    "fcmoe_bf16_forward": (_I, [ctypes.POINTER(MoeArgs), _P]),
    "fcmoe_w8a16_workspace_bytes": (_SZ, [ctypes.POINTER(MoeArgs)]),
    "fcmoe_w8a16_forward": (_I, [ctypes.POINTER(MoeArgs), _P]),
    "fcmoe_i8gemm_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "fcmoe_i8gemm_pair_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "fcmoe_i8gemm": (_I, [_P, _I, _I64, _I64, _P, _P, _I64, _P, _P, _I, _P, _SZ, _P]),
    "fcmoe_i8gemm_pair": (_I, [_P, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _SZ, _P]),
    "fcmoe_grouped_gemm_i8_acc": (_I, [_P, _I64, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _P, _P, _SZ, _P]),
    "fcmoe_grouped_gemm_workspace_bytes": (_SZ, [_I64, _I64]),
    "fcmoe_w8a8_stage_views": (_I, [ctypes.POINTER(MoeArgs), _P, _P, _P, _P, _P, _P, _P]),
    "fcmoe_bf16_stage_views": (_I, [ctypes.POINTER(MoeArgs), _I, _P, _P, _P]),
    "fcmoe_stage_timing_enable": (_I, [_I]),
    "fcmoe_stage_timing_read": (_I, [_P, _P]),
    "fcmoe_w8a8_prefill_plan": (_I, [_P, _P]),
}

FCMOE_STAGE_COUNT = 24
FCMOE_NOALLOC_SCRATCH_BYTES = 64 << 20
STAGE_NAMES = {0: "route", 1: "quant", 2: "requant", 3: "act", 4: "combine",
               **{8 + c: f"w13_bm{bm}" for c, bm in enumerate((16, 32, 64, 128, 192, 256))},
               **{16 + c: f"w2_bm{bm}" for c, bm in enumerate((16, 32, 64, 128, 192, 256))},
               14: "w13_mixed_mfma", 15: "w13_mixed_stream", 22: "w2_mixed_mfma", 23: "w2_mixed_stream"}


def stage_timing_enable(on: bool = True) -> None:
    check(lib().fcmoe_stage_timing_enable(1 if on else 0), "stage_timing_enable")


def stage_timing_read() -> dict[str, tuple[float, int]]:
    """{stage name: (total ms, launches)} since the last read; clears the records."""
    ms = (ctypes.c_double * FCMOE_STAGE_COUNT)()
    n = (ctypes.c_int64 * FCMOE_STAGE_COUNT)()
    check(lib().fcmoe_stage_timing_read(ctypes.cast(ms, ctypes.c_void_p), ctypes.cast(n, ctypes.c_void_p)),
          "stage_timing_read")
    return {STAGE_NAMES[i]: (ms[i], n[i]) for i in range(FCMOE_STAGE_COUNT) if n[i] > 0}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built (python -m fused_cpp_amd.build)")
        l = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {lib().fcmoe_last_error().decode()}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle() -> int:
    import torch

    return torch.cuda.current_stream().cuda_stream


def w8a8_prefill_plan(class_tiles) -> tuple[str, int]:
    """The W8A8 prefill launch plan the device picks for these per-class tile
    counts (16 / 128 / 192 / 256 rows): ("classic" | "mixed" | "partitioned",
    CUs of the partitioned 256-row class)."""
    tiles = (ctypes.c_int32 * 4)(*[int(t) for t in class_tiles])
    wgs = ctypes.c_int(0)
    rc = lib().fcmoe_w8a8_prefill_plan(ctypes.cast(tiles, ctypes.c_void_p), ctypes.byref(wgs))
    check(rc if rc < 0 else 0, "w8a8_prefill_plan")
    return ("classic", "mixed", "partitioned")[rc], wgs.value
