"""Capacity tiers of the fixed-shape graphs (fastmd/engine/capacity_policy.py:19-24, 211-214,
267-316 of the reference): a capture holds ``tier(held_demand(demand))`` undirected pairs and
grows monotonically when a window overflows."""
from __future__ import annotations

from dataclasses import dataclass

GROWTH_HEADROOM = 1 / 128


def tier(value: int, step: int, min_pad: int) -> int:
    """The next multiple of ``step`` above ``value``, one more step if that leaves less than
    ``min_pad`` slack."""
    capacity = (int(value) // step + 1) * step
    return capacity + step if capacity - int(value) < min_pad else capacity


def held_demand(demand: int, headroom: int, factor: float) -> int:
    """demand + headroom, or for a declared thermal factor the larger of that and factor * demand."""
    return demand + headroom if factor == 1.0 else max(demand + headroom, int(round(demand * factor)))


def whole_step_headroom(demand: int, step: int, fraction: float = GROWTH_HEADROOM) -> int:
    """Headroom of a whole-step capture: the growth fraction in whole steps (gpu_md.py:764-772)."""
    return int(demand * fraction) // step * step


@dataclass(frozen=True)
class CapacityKey:
    u_capacity: int
    t_capacity: int = 0


class JointCapacityPolicy:
    """Edges-only capacity tiers with monotonic growth (capacity_policy.py:267-316)."""

    def __init__(self, *, u_step: int = 512, min_pad_u: int = 256) -> None:
        self.u_step, self.min_pad_u = int(u_step), int(min_pad_u)
        self.capacity_history: list[CapacityKey] = []

    def key_for(self, u: int) -> CapacityKey:
        return CapacityKey(tier(u, self.u_step, self.min_pad_u), 0)

    def start(self, u: int) -> CapacityKey:
        key = self.key_for(u)
        self.capacity_history.append(key)
        return key

    def grow(self, current: CapacityKey, u: int) -> CapacityKey:
        grown = CapacityKey(max(current.u_capacity, self.key_for(u).u_capacity), 0)
        if grown != current:
            self.capacity_history.append(grown)
        return grown
