"""Plan V2 schema compatibility (src/fused_cpp/moe/plan.py:11-461).

The reference executes W8A8/BF16 MoE through CPU thread plans. On MI355X the
work decomposition is chosen on the GPU from the per-expert token counts, so a
plan carries no information the kernels use: plans are accepted, their schema
is validated, and they are otherwise ignored.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping

import torch

ASYNC_MOE_PLAN_VERSION = 2
ASYNC_MOE_EXECUTION_STRICT = "strict"
ASYNC_MOE_EXECUTION_TAIL_POOL = "tail_pool"
ASYNC_MOE_PLACEMENT_FIXED = 0
ASYNC_MOE_PLACEMENT_TAIL_POOL = 1
ASYNC_MOE_STAGE_EXPERT = 0
ASYNC_MOE_RESIZE_NONE = 0
ASYNC_MOE_FULL_EXPERT_RANGE = 0

_SEQUENCE_FIELDS = (
    "thread_cpu_ids",
    "task_expert_ids",
    "task_core_begins",
    "task_threads",
    "task_dep_offsets",
    "task_deps",
    "task_preferred_threads",
    "task_min_threads",
    "task_max_threads",
    "task_allowed_thread_offsets",
    "task_allowed_threads",
    "task_placement_modes",
    "task_numa_nodes",
    "task_stage_ids",
    "task_resize_points",
    "task_range_granularities",
)
_OPTIONAL_PER_TASK = ("task_w13_window_tiles", "task_w2_window_tiles")


def _int_tensor(value: object, name: str) -> torch.Tensor:
    tensor = value if isinstance(value, torch.Tensor) else torch.as_tensor(value, dtype=torch.int64)
    if tensor.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64):
        raise TypeError(f"{name} must use an integer dtype, got {tensor.dtype}")
    if tensor.dim() != 1:
        raise ValueError(f"{name} must be 1-D")
    return tensor.to(torch.int64)


@dataclass(frozen=True)
class AsyncMoEPlanV2:
    """Validated Plan V2 bridge (fields as in the reference); execution ignores it."""

    num_threads: int
    execution_mode: str
    thread_cpu_ids: torch.Tensor
    task_expert_ids: torch.Tensor
    task_core_begins: torch.Tensor
    task_threads: torch.Tensor
    task_dep_offsets: torch.Tensor
    task_deps: torch.Tensor
    task_preferred_threads: torch.Tensor
    task_min_threads: torch.Tensor
    task_max_threads: torch.Tensor
    task_allowed_thread_offsets: torch.Tensor
    task_allowed_threads: torch.Tensor
    task_placement_modes: torch.Tensor
    task_numa_nodes: torch.Tensor
    task_stage_ids: torch.Tensor
    task_resize_points: torch.Tensor
    task_range_granularities: torch.Tensor
    task_w13_window_tiles: torch.Tensor | None = None
    task_w2_window_tiles: torch.Tensor | None = None
    early_merge: bool | None = None

    @property
    def plan_version(self) -> int:
        return ASYNC_MOE_PLAN_VERSION

    @property
    def native_execution_mode(self) -> int:
        return {ASYNC_MOE_EXECUTION_STRICT: 0, ASYNC_MOE_EXECUTION_TAIL_POOL: 1}[self.execution_mode]

    @property
    def native_early_merge(self) -> int:
        return -1 if self.early_merge is None else int(self.early_merge)

    def __post_init__(self) -> None:
        tasks = int(self.task_expert_ids.numel())
        for name in _OPTIONAL_PER_TASK:
            if getattr(self, name) is None:
                object.__setattr__(self, name, torch.zeros(tasks, dtype=torch.int64))
        self.validate()

    def validate(self) -> None:
        if self.execution_mode not in (ASYNC_MOE_EXECUTION_STRICT, ASYNC_MOE_EXECUTION_TAIL_POOL):
            raise ValueError(f"unknown execution_mode {self.execution_mode!r}")
        if int(self.num_threads) <= 0:
            raise ValueError("num_threads must be positive")
        tasks = int(self.task_expert_ids.numel())
        for name in ("task_core_begins", "task_threads", "task_min_threads", "task_max_threads"):
            if int(getattr(self, name).numel()) != tasks:
                raise ValueError(f"{name} must have one entry per task")
        if int(self.task_dep_offsets.numel()) != tasks + 1:
            raise ValueError("task_dep_offsets must have tasks + 1 entries")

    @classmethod
    def from_dict(cls, plan: Mapping[str, object]) -> "AsyncMoEPlanV2":
        version = int(plan.get("plan_version", -1))  # type: ignore[arg-type]
        if version != ASYNC_MOE_PLAN_VERSION:
            raise ValueError(f"plan_version must be {ASYNC_MOE_PLAN_VERSION}, got {version}")
        required = ("num_threads", "execution_mode", *_SEQUENCE_FIELDS)
        missing = [name for name in required if name not in plan]
        if missing:
            raise ValueError(f"Plan V2 is missing required fields: {', '.join(missing)}")
        tensors = {name: _int_tensor(plan[name], name) for name in _SEQUENCE_FIELDS}
        tasks = int(tensors["task_expert_ids"].numel())
        for name in _OPTIONAL_PER_TASK:
            tensors[name] = _int_tensor(plan.get(name, [0] * tasks), name)
        early = plan.get("early_merge")
        if early is not None and type(early) is not bool:
            raise TypeError("early_merge must be a bool or None")
        return cls(num_threads=int(plan["num_threads"]), execution_mode=str(plan["execution_mode"]),
                   early_merge=early, **tensors)


def upgrade_legacy_async_plan(plan: Mapping[str, object]) -> dict[str, object]:
    """Fill the strict Plan V2 fields of a legacy fixed-width bridge."""
    widths = [int(w) for w in plan["task_threads"]]  # type: ignore[union-attr]
    tasks = len(widths)
    upgraded = dict(plan)
    upgraded.update(
        plan_version=ASYNC_MOE_PLAN_VERSION,
        execution_mode=ASYNC_MOE_EXECUTION_STRICT,
        task_preferred_threads=list(widths),
        task_min_threads=list(widths),
        task_max_threads=list(widths),
        task_allowed_thread_offsets=list(range(tasks + 1)),
        task_allowed_threads=list(widths),
        task_placement_modes=[ASYNC_MOE_PLACEMENT_FIXED] * tasks,
        task_numa_nodes=[-1] * tasks,
        task_stage_ids=[ASYNC_MOE_STAGE_EXPERT] * tasks,
        task_resize_points=[ASYNC_MOE_RESIZE_NONE] * tasks,
        task_range_granularities=[ASYNC_MOE_FULL_EXPERT_RANGE] * tasks,
        early_merge=None,
    )
    return upgraded


def materialize_plan(plan: object) -> AsyncMoEPlanV2:
    return plan if isinstance(plan, AsyncMoEPlanV2) else AsyncMoEPlanV2.from_dict(plan)  # type: ignore[arg-type]


__all__ = [
    "ASYNC_MOE_EXECUTION_STRICT",
    "ASYNC_MOE_EXECUTION_TAIL_POOL",
    "ASYNC_MOE_FULL_EXPERT_RANGE",
    "ASYNC_MOE_PLACEMENT_FIXED",
    "ASYNC_MOE_PLACEMENT_TAIL_POOL",
    "ASYNC_MOE_PLAN_VERSION",
    "ASYNC_MOE_RESIZE_NONE",
    "ASYNC_MOE_STAGE_EXPERT",
    "AsyncMoEPlanV2",
    "upgrade_legacy_async_plan",
]
