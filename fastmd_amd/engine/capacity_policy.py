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
    """Pair (and, with a triplet step, triplet) capacity tiers with monotonic growth
    (capacity_policy.py:267-316): each count takes its own tier, growth keeps the larger."""

    def __init__(self, *, u_step: int = 512, min_pad_u: int = 256, t_step: int | None = None,
                 min_pad_t: int | None = None) -> None:
        self.u_step, self.min_pad_u = int(u_step), int(min_pad_u)
        self.t_step = None if t_step is None else int(t_step)
        self.min_pad_t = int(min_pad_t if min_pad_t is not None else (t_step or 0))
        self.capacity_history: list[CapacityKey] = []

    def key_for(self, u: int, t: int = 0) -> CapacityKey:
        return CapacityKey(tier(u, self.u_step, self.min_pad_u),
                           tier(t, self.t_step, self.min_pad_t) if self.t_step else 0)

    def start(self, u: int, t: int = 0) -> CapacityKey:
        key = self.key_for(u, t)
        self.capacity_history.append(key)
        return key

    def grow(self, current: CapacityKey, u: int, t: int = 0) -> CapacityKey:
        want = self.key_for(u, t)
        grown = CapacityKey(max(current.u_capacity, want.u_capacity), max(current.t_capacity, want.t_capacity))
        if grown != current:
            self.capacity_history.append(grown)
        return grown
