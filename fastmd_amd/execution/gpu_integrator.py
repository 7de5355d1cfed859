"""Integrator protocol of the GPU-resident MD step and the sync-free constant upload.

``StatefulIntegrator`` mirrors the reference's protocol (fastmd/execution/gpu_integrator.py:69-191):
the integrator owns the authoritative float64 MD state and splits a step into
``step_pre_force`` (returns q_{n+1}) and ``step_post_force(F, energy)``, with a one-copy
backup/restore transaction and snapshots. ``_PinnedUpload`` (:34-66) rewrites a small device
constant vector from pinned host memory, stream ordered, without a host sync.
"""
from __future__ import annotations

from typing import Protocol, runtime_checkable

import torch
from torch import Tensor


def kinetic_energy_fp64(momenta: Tensor, masses: Tensor) -> Tensor:
    """0.5 * sum(p * (p / m)) in float64 (gpu_integrator.py:12-21)."""
    p = momenta.to(torch.float64)
    return 0.5 * (p * (p / masses.to(torch.float64).reshape(-1, 1))).sum()


class _PinnedUpload:
    """Sync-free host -> device rewrite of a small float64 vector (gpu_integrator.py:34-66).

    Two pinned slots alternate, so a slot is never rewritten while a previous copy from it may
    still be in flight; an event per slot orders the reuse. Raises inside a graph capture (the
    host values would be baked into the graph)."""

    def __init__(self, target: Tensor) -> None:
        self.target = target
        self.slots = [torch.empty(target.shape, dtype=target.dtype, pin_memory=True) for _ in range(2)]
        self.events = [None, None]
        self.next = 0

    def __call__(self, values) -> None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("set_temperature inside a graph capture: call it between replays")
        k = self.next
        self.next = 1 - k
        if self.events[k] is not None:
            self.events[k].synchronize()
        self.slots[k].copy_(torch.as_tensor(values, dtype=self.target.dtype).reshape(self.target.shape))
        self.target.copy_(self.slots[k], non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        self.events[k] = event


@runtime_checkable
class StatefulIntegrator(Protocol):
    """The integrator of a whole-step window (gpu_integrator.py:69-191)."""

    def step_pre_force(self) -> Tensor: ...

    def step_post_force(self, forces: Tensor, energy: Tensor | None = None) -> None: ...

    def set_forces(self, forces, energy=None) -> None: ...

    def backup(self, state=None) -> None: ...  # state (default: the live one) into the backup

    def restore(self, state=None) -> None: ...  # the backup into state (default: the live one)

    def new_state(self): ...  # a state of the same shape (the runner's held window start)

    def snapshot(self) -> tuple: ...

    def load_snapshot(self, snapshot: tuple) -> None: ...
