"""Public inference configuration of the GPU-resident MD step.

Field names and meanings of the reference's ``CapacityConfig`` and the execution switch of
``InferenceConfig`` (fastmd/config.py:433-601); the MatRIS-specific expert options are out of
scope. ``optimization_profile="generic"`` of the reference selects its plain-torch reference
operators; here the plain reference is the CPU oracle (tests only), so the profile is accepted
for signature parity and the HIP kernels always run.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

EXECUTION_MODES = ("auto", "eager", "model_graph", "whole_step")


@dataclass(frozen=True)
class CapacityConfig:
    u_step: int = 512
    t_step: int = 8192
    n_dummy: int = 64
    min_pad_u: int = 256
    min_pad_t: int = 4096
    warmup: int = 3
    candidate_skin: float = 2.0

    def __post_init__(self) -> None:
        for name in ("u_step", "t_step", "n_dummy", "min_pad_u", "min_pad_t", "warmup"):
            minimum = 1 if name in {"u_step", "t_step", "n_dummy"} else 0
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int) or value < minimum:
                raise ValueError(f"capacity.{name} must be an integer >= {minimum}")
        skin = self.candidate_skin
        if isinstance(skin, bool) or not isinstance(skin, (int, float)) or not math.isfinite(skin) or skin < 0:
            raise ValueError("capacity.candidate_skin must be finite and >= 0 angstrom")


@dataclass(frozen=True)
class InferenceConfig:
    execution: str | None = "auto"
    optimization_profile: str | None = None
    capacity: CapacityConfig = field(default_factory=CapacityConfig)

    def __post_init__(self) -> None:
        if self.execution is not None and self.execution not in EXECUTION_MODES:
            raise ValueError(f"execution must be one of {EXECUTION_MODES}, got {self.execution!r}")
        if self.optimization_profile not in (None, "topology", "generic", "legacy"):
            raise ValueError(f"unknown optimization_profile {self.optimization_profile!r}")
        if not isinstance(self.capacity, CapacityConfig):
            raise TypeError("capacity must be a CapacityConfig")

    @property
    def resolved_execution(self) -> str:
        """The mode a run starts in: "auto" starts whole-step; the driver falls back to eager
        on an out-of-memory error in a whole-step capture (gpu_md.py:1720-1774)."""
        return "whole_step" if self.execution in (None, "auto") else self.execution
