"""CPU oracle molecular dynamics for the MD tests and the golden-fixture generator (test
infrastructure; not collected by pytest).

Force fields evaluate the oracle models (``oracle/models.py``) on pair lists formed here by brute
force over the 27 neighbouring images, independently of the neighbour-list oracle: candidate pairs
within rc + skin are listed from the wrapped positions and listed again once an atom has moved
more than skin / 2 since the last listing (the reference's skin rule,
fastmd/execution/whole_step_cuda_graph.py:579-584); every evaluation keeps the pairs with
r < rc in float64. Forces are returned as float32, like the GPU model's, so that the NHC kick has
the reference's float32 semantics (fastmd/execution/gpu_nhc.py:380-384). The integrator is the
NHC oracle (``oracle/nhc.py``). A system's cell must be wider than 2 (rc + skin) along each
height so that the 27 images hold every pair once.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import models as om
from oracle import nhc as onhc

SHIFTS = np.array([[a, b, c] for a in (-1, 0, 1) for b in (-1, 0, 1) for c in (-1, 0, 1)], dtype=np.int64)


class PairList:
    """Candidate pairs (i, j, image) within ``rc + skin`` with the skin refresh rule; ``pairs(q)``
    returns the float64 edge rows (centre i, neighbour j, integer image in the frame of the
    unwrapped positions q) with r < rc."""

    def __init__(self, cell, rc: float = 6.0, skin: float = 2.0) -> None:
        self.cell = np.asarray(cell, dtype=np.float64)
        self.inv = np.linalg.inv(self.cell)
        self.rc, self.skin = float(rc), float(skin)
        heights = 1.0 / np.linalg.norm(self.inv, axis=0)
        if np.any(heights < 2 * (self.rc + self.skin)):
            raise ValueError("cell too small for a 27-image pair list")
        self.q0 = None
        self.listings = 0

    def _list(self, q):
        wraps = np.floor(q @ self.inv)
        w = q - wraps @ self.cell
        d = w[None, :, None, :] + (SHIFTS @ self.cell)[None, None, :, :] - w[:, None, None, :]
        r = np.linalg.norm(d, axis=-1)
        ii, jj, kk = np.nonzero((r < self.rc + self.skin) & (r > 1e-8))
        # image of the pair in the frame of the unwrapped positions
        img = SHIFTS[kk] - wraps[jj].astype(np.int64) + wraps[ii].astype(np.int64)
        self.q0, self.ii, self.jj, self.img = q.copy(), ii, jj, img
        self.listings += 1

    def pairs(self, q):
        if self.q0 is None or np.max(np.linalg.norm(q - self.q0, axis=1)) >= self.skin / 2:
            self._list(q)
        vec = q[self.jj] + self.img @ self.cell - q[self.ii]
        keep = np.linalg.norm(vec, axis=1) < self.rc
        return self.ii[keep], self.jj[keep], self.img[keep]


def morse_forces(system, rc: float = 6.0, skin: float = 2.0):
    """configs[0]'s shifted Morse pair potential (oracle ``morse_node_energy``), vectorized."""
    plist = PairList(system.cell, rc, skin)
    cell = np.asarray(system.cell, dtype=np.float64)
    D, a, r0 = 0.3, 1.5, 3.0
    vrc = D * ((1 - np.exp(-a * (rc - r0))) ** 2 - 1)

    def forces(q):
        ii, jj, img = plist.pairs(q)
        dv = q[jj] + img @ cell - q[ii]
        rr = np.linalg.norm(dv, axis=1)
        ex = np.exp(-a * (rr - r0))
        v = D * ((1 - ex) ** 2 - 1) - vrc
        fij = (0.5 * 2 * D * (1 - ex) * a * ex / rr)[:, None] * dv  # each pair is listed as i-j and j-i
        f = np.zeros_like(q)
        np.add.at(f, ii, fij)
        np.add.at(f, jj, -fij)
        return f.astype(np.float32), 0.5 * float(v.sum())

    forces.pair_list = plist
    return forces


def mace_like_forces(system, params: dict, config: dict, rc: float = 6.0, skin: float = 2.0,
                     dtype=torch.float64):
    """The MACE-like oracle model (``mace_like_node_energy`` differentiated by the engine-owned
    derivative, ``energy_and_forces``: float64 energy sum) on the skin pair list, evaluated on the
    wrapped positions (as the reference's builder publishes them, fixed_capacity_builder.py:
    2260-2282) in ``dtype``: float64 for the exact trajectory, float32 for the arithmetic class
    of the reference's own model path."""
    plist = PairList(system.cell, rc, skin)
    elem_of = {z: k for k, z in enumerate(config["elements"])}
    elem = torch.tensor([elem_of[int(z)] for z in system.numbers])
    cell_np = np.asarray(system.cell, dtype=np.float64)
    cell = torch.tensor(cell_np, dtype=dtype)
    inv = np.linalg.inv(cell_np)

    def forces(q):
        ii, jj, img = plist.pairs(q)
        wraps = np.floor(q @ inv).astype(np.int64)
        wrapped = q - wraps @ cell_np
        img = img + wraps[jj] - wraps[ii]  # the same pair in the frame of the wrapped positions
        order = np.lexsort((jj, ii))  # receiver-sorted rows, as the GPU's canonical list
        center, neighbor = torch.tensor(ii[order]), torch.tensor(jj[order])
        images = torch.tensor(img[order].astype(np.int32))
        energy, f, _ = om.energy_and_forces(
            lambda pos: om.mace_like_node_energy(params, config, pos, cell, elem, center, neighbor, images),
            torch.tensor(wrapped, dtype=dtype))
        return f.numpy().astype(np.float32), float(energy)

    forces.pair_list = plist
    return forces


def run_nhc(system, forces, momenta, steps: int, *, sample_every: int = 10, positions_until: int = 0,
            temperature: float = 500.0, timestep_fs: float = 0.25, tdamp_fs: float = 25.0, progress=None):
    """Integrate ``steps`` NHC steps (tchain 3, tloop 1, float32 kick) from the system's positions
    and ``momenta``. Returns the conserved quantity C(t) at t = 0, sample_every, ... and, at the
    sampled steps up to ``positions_until``, the positions, momenta, forces and potential energy."""
    f0, e0 = forces(system.positions)
    o = onhc.NHC(system.masses, system.positions, momenta, temperature_K=temperature,
                 timestep=timestep_fs * onhc.FS, tdamp=tdamp_fs * onhc.FS, f32_kick=True, forces=f0, energy=e0)
    steps_at, conserved = [0], [o.conserved_energy()]
    states = {"positions": [o.q.copy()], "momenta": [o.p.copy()], "forces": [o.f.copy()], "energy": [o.e]}
    for k in range(1, steps + 1):
        o.step(forces)
        if k % sample_every == 0:
            steps_at.append(k)
            conserved.append(o.conserved_energy())
            if k <= positions_until:
                for key, value in (("positions", o.q), ("momenta", o.p), ("forces", o.f), ("energy", o.e)):
                    states[key].append(np.copy(value))
            if progress is not None and k % (100 * sample_every) == 0:
                progress(k)
    return {"steps": np.array(steps_at), "conserved": np.array(conserved),
            **{key: np.array(value) for key, value in states.items()}}


def max_drift(conserved) -> float:
    """max_t |C(t) - C(0)| over the sampled steps."""
    c = np.asarray(conserved, dtype=np.float64)
    return float(np.max(np.abs(c - c[0])))
