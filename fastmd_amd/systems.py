"""Synthetic periodic systems of the benchmark configurations (seeded, NumPy only).

Cubic ABX3 perovskite supercells: lattice constant ``a`` per 5-atom cell, fractional sites
A (0,0,0), B (1/2,1/2,1/2), X (1/2,1/2,0), (1/2,0,1/2), (0,1/2,1/2) (the geometry of the
reference's MACE adapter fixture, tests/adapters/test_mace_adapter.py:139-148, without its
shear), masses A/B/X = 133/119/127 amu (Cs/Sn/I numbers 55/50/53), Gaussian jitter of
``sigma`` Angstrom from ``numpy.random.default_rng(seed)``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

_SITES = np.array([[0.0, 0.0, 0.0], [0.5, 0.5, 0.5], [0.5, 0.5, 0.0], [0.5, 0.0, 0.5], [0.0, 0.5, 0.5]])
_NUMBERS = np.array([55, 50, 53, 53, 53], dtype=np.int32)
_MASSES = {55: 133.0, 50: 119.0, 53: 127.0}


@dataclass
class System:
    positions: np.ndarray  # float64 [N, 3], Angstrom
    cell: np.ndarray  # float64 [3, 3], rows are lattice vectors
    numbers: np.ndarray  # int32 [N]
    masses: np.ndarray  # float64 [N], amu

    @property
    def n_atoms(self) -> int:
        return int(self.positions.shape[0])


def perovskite(repeats=(3, 3, 3), a: float = 6.2, sigma: float = 0.05, seed: int = 0) -> System:
    """``repeats`` cells per axis (an int for k x k x k): N = 5 * product(repeats)."""
    if isinstance(repeats, int):
        repeats = (repeats, repeats, repeats)
    r = np.asarray(repeats, dtype=np.int64)
    grid = np.stack(np.meshgrid(*[np.arange(k) for k in r], indexing="ij"), -1).reshape(-1, 3)
    frac = (grid[:, None, :] + _SITES[None, :, :]).reshape(-1, 3) / r[None, :]
    cell = np.diag(r.astype(np.float64) * a)
    positions = frac @ cell
    rng = np.random.default_rng(seed)
    positions = positions + rng.normal(0.0, sigma, positions.shape)
    numbers = np.tile(_NUMBERS, int(np.prod(r)))
    masses = np.array([_MASSES[int(z)] for z in numbers], dtype=np.float64)
    return System(positions, cell, numbers, masses)


def perovskite_atoms(n_atoms: int, **kwargs) -> System:
    """The supercells the configurations name by atom count: 135 = 3x3x3, 3 430 = 7x7x14,
    10 000 = 10x10x20, 5k^3 otherwise."""
    special = {3430: (7, 7, 14), 10000: (10, 10, 20)}
    if n_atoms in special:
        return perovskite(special[n_atoms], **kwargs)
    k = round((n_atoms / 5) ** (1 / 3))
    if 5 * k ** 3 != n_atoms:
        raise ValueError(f"no perovskite supercell of {n_atoms} atoms")
    return perovskite(k, **kwargs)
