"""Loader for the compiled host extension and the C-ABI library.

There is no fallback: if ``_moe_C`` (the torch extension over libfcmoe.so) is
missing, every operator raises ``RuntimeError`` naming the build command.
"""

from __future__ import annotations

import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libfcmoe.so"

try:  # pragma: no cover - exercised by the import itself
    from fused_cpp_amd import _moe_C as moe_C  # type: ignore[attr-defined]

    NATIVE_ERROR: str | None = None
except ImportError as error:  # pragma: no cover
    moe_C = None
    NATIVE_ERROR = f"{error}"


def require_native():
    """Return the extension module or raise with the build instruction."""
    if moe_C is None:
        raise RuntimeError(
            "fused_cpp_amd native extension is not built (python -m fused_cpp_amd.build): " + str(NATIVE_ERROR)
        )
    return moe_C


def gpu_available() -> bool:
    """True when a ROCm device is visible (device_count does not initialise HIP)."""
    import torch

    if os.environ.get("FUSED_CPP_AMD_FORCE_NO_GPU") == "1":
        return False
    return bool(torch.version.hip) and torch.cuda.device_count() > 0


def validate_ids_default() -> bool:
    """Range-check topk_ids in each call, as the reference does on the host
    (csrc/moe/arm/i8mm_w8a8/kernels.cpp:583-587): the route launch writes the
    count of invalid ids to pinned host memory, which the call polls until the
    route launch has written it (the rest of the forward keeps running; no
    measurable cost per call at one token or at 64). Set
    FUSED_CPP_AMD_VALIDATE_IDS=0 to skip the check.
    The read is skipped while the current stream is being captured into a
    HIP graph (a host read cannot be captured; invalid ids then contribute
    nothing, as with the variable set to 0)."""
    if os.environ.get("FUSED_CPP_AMD_VALIDATE_IDS", "1") == "0":
        return False
    import torch

    if not torch.cuda.is_initialized():
        return True  # nothing can be capturing before the device is initialised
    return not torch.cuda.is_current_stream_capturing()
