"""Candidate-list sizing shared by the builders.

The reference sizes its candidate rows with nvalchemiops' estimate
(fastmd/graph/neighbor_list_backend.py:77-88) and raises ``NeighborOverflowError`` when a row
was truncated; the cell list itself is this package's HIP kernel (``fmd_nl_candidates``),
so there is no third-party backend to select.
"""
from __future__ import annotations

import math

import numpy as np


class NeighborOverflowError(RuntimeError):
    """A candidate row held more candidates than its slots (the refresh must be redone with more)."""

    def __init__(self, capacity: int, max_count: int) -> None:
        super().__init__(f"neighbor list overflow: {max_count} candidates for {capacity} slots")
        self.capacity = capacity
        self.max_count = max_count


def estimate_max_neighbors(cutoff: float, atomic_density: float = 0.35, safety_factor: float = 5.0) -> int:
    """``safety_factor * atomic_density * (4/3) pi cutoff^3``, at least 1, rounded up to a
    multiple of 16; 0 for a non-positive cutoff (neighbor_list_backend.py:77-88)."""
    if cutoff <= 0:
        return 0
    volume = atomic_density * (4.0 / 3.0) * math.pi * (cutoff ** 3)
    expected = max(1, safety_factor * volume)
    return int(math.ceil(expected / 16)) * 16


def cell_heights(cell) -> np.ndarray:
    """Perpendicular heights of the cell (volume / face area per axis)."""
    c = np.asarray(cell, dtype=np.float64)
    volume = abs(np.linalg.det(c))
    return np.array([volume / np.linalg.norm(np.cross(c[(k + 1) % 3], c[(k + 2) % 3])) for k in range(3)])


def cell_list_shape(cell, cutoff: float) -> tuple[tuple[int, int, int], tuple[int, int, int]]:
    """Cells per lattice axis (slabs at least ``cutoff`` thick) and the search reach per axis:
    a pair within the cutoff is at most ``floor(cutoff * n / h) + 1`` cells apart along an axis of
    perpendicular height h split into n slabs (one cell of margin for rounding at slab edges)."""
    heights = cell_heights(cell)
    if not np.all(heights > 0):
        raise ValueError("degenerate cell")
    ncells = tuple(int(max(1, math.floor(h / cutoff))) for h in heights)
    reach = tuple(int(math.floor(cutoff * n / h)) + 1 for n, h in zip(ncells, heights))
    return ncells, reach
