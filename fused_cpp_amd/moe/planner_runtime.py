"""Planner runtime compatibility (src/fused_cpp/moe/planner_runtime.py:35-401).

The reference plans CPU thread teams per call. On MI355X the grouped-GEMM tile
classes are selected on the GPU from the per-expert token counts inside the
operator, so the runtime only needs to exist for callers' initialisation code:
it is constructible, installable and returns no plans. No calibration runs.
"""

from __future__ import annotations

import tempfile
import threading
from pathlib import Path
from typing import Any, Sequence

DEFAULT_MOE_COST_CACHE_DIR = Path(tempfile.gettempdir()) / "fused_cpp_amd_moe_cost_cache"

_lock = threading.Lock()
_default_runtime: "MoePlannerRuntime | None" = None


class MoePlannerRuntime:
    """Accepts the reference constructor arguments; plans are selected on the GPU."""

    def __init__(self, calibration: Any = None, *, hidden_size: int, intermediate_size: int, global_experts: int,
                 local_experts: int, mode: str = "standalone", degree: int = 1, concurrent_ranks: int = 1,
                 cpu_ids: Sequence[int] | None = None, shared_experts: int = 0,
                 cost_cache_dir: str | Path | None = DEFAULT_MOE_COST_CACHE_DIR) -> None:
        if int(shared_experts) not in (0, 1):
            raise ValueError("shared_experts must be 0 or 1")
        self.calibration = calibration
        self.hidden_size = int(hidden_size)
        self.intermediate_size = int(intermediate_size)
        self.global_experts = int(global_experts)
        self.local_experts = int(local_experts)
        self.shared_experts = int(shared_experts)
        self._last_plan: dict[str, object] = {}

    def initialize_planner(self, max_routes: int) -> dict[str, object]:
        return {"max_routes": int(max_routes), "selector": "gpu_tile_classes"}

    def plan_for_dispatch(self, weights: Any, topk_ids: Any, **kwargs: Any) -> None:
        """No CPU plan: the GPU operator selects its tiles from the routed counts."""
        return None

    def plan_for_shared_dispatch(self, weights: Any, combined_ids: Any, **kwargs: Any) -> None:
        return None

    def last_plan(self) -> dict[str, object]:
        return dict(self._last_plan)


def set_default_moe_planner_runtime(runtime: MoePlannerRuntime | None) -> MoePlannerRuntime | None:
    if runtime is not None and not isinstance(runtime, MoePlannerRuntime):
        raise TypeError("runtime must be a MoePlannerRuntime or None")
    global _default_runtime
    with _lock:
        previous, _default_runtime = _default_runtime, runtime
        return previous


def get_default_moe_planner_runtime() -> MoePlannerRuntime | None:
    with _lock:
        return _default_runtime


def calibrate_moe_planner_quick(*args: Any, **kwargs: Any) -> None:
    """There is no CPU cost model to calibrate on this backend."""
    return None


def enable_moe_planner_quick(*, hidden_size: int, intermediate_size: int, global_experts: int, local_experts: int,
                             shared_experts: int = 0, **kwargs: Any) -> MoePlannerRuntime:
    runtime = MoePlannerRuntime(None, hidden_size=hidden_size, intermediate_size=intermediate_size,
                                global_experts=global_experts, local_experts=local_experts,
                                shared_experts=shared_experts)
    set_default_moe_planner_runtime(runtime)
    return runtime


__all__ = [
    "DEFAULT_MOE_COST_CACHE_DIR",
    "MoePlannerRuntime",
    "calibrate_moe_planner_quick",
    "enable_moe_planner_quick",
    "get_default_moe_planner_runtime",
    "set_default_moe_planner_runtime",
]
