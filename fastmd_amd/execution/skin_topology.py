"""Skin-epoch topology reuse for fixed-frame evaluations of one periodic system
(fastmd/execution/skin_topology.py:97-442, ``SkinTopologyRunner``).

A calculator that rebuilds the ragged graph on every call pays host synchronizations while the GPU
idles. Here one owner builder keeps the candidate list (cutoff rc + skin) across calls, and every
call runs the exact device re-filter of those candidates (d < rc, plus the line graph for a
three-body model) into a padded bucket, then the model's forward and VJP. With ``capture`` the
build and the model are one hipGraph per capacity bucket. A call is: copy the positions in, one
replay (or the eager body), one readback of the energy, the forces and a status vector.

Exactness: the candidate list is the only topology state carried between calls.
* The host refreshes it before the launch once an atom moved ``PROACTIVE_REFRESH_FRACTION`` of the
  skin since the last refresh. That displacement is the minimum image, so a caller's lattice wrap
  is no motion; the builders run with ``minimum_image`` for the same reason.
* The device checks on every call that no atom moved half the skin (2 max|d| <= skin); then every
  pair within rc is a candidate.
* A stale list is refreshed and the call redone. A capacity overflow (the bucket evaluated its
  padding) is redone in a bucket that holds the counts the overflowing build reported.
* A truncated candidate row raises ``SkinTopologyUnavailable``: the caller goes back to the per-call
  rebuild.

Buckets are keyed (u_cap, t_cap) with the model_graph runner's capacity rule (``tier`` of the
demand held above the last count); the demand of a call is the previous call's counts plus the
minimum padding, or the exact count at a refresh.
"""
from __future__ import annotations

import numpy as np
import torch

from fastmd_amd._roctx import roctx_range
from fastmd_amd.adapters.protocol import PaddingRule
from fastmd_amd.engine.capacity_policy import held_demand, tier
from fastmd_amd.engine.energy_derivative import engine_derivative
from fastmd_amd.execution.graph_capture import capture_graph
from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder, fixed_capacity_exceeded

# The host refreshes the candidates before the launch once an atom moved this fraction of the skin
# (0.9 of the device's limit of half the skin: the margin covers the host's float64 vs the
# device's float32 arithmetic).
PROACTIVE_REFRESH_FRACTION = 0.45
# Evaluations of one call: the first, a refresh, a growth and one spare.
MAX_ATTEMPTS = 4


class SkinTopologyUnavailable(RuntimeError):
    """The candidate list cannot hold this system (a truncated row): rebuild per call instead."""


class SkinTopologyRunner:
    """Energy and forces of one periodic system at host coordinates, with a skin-epoch topology.

    ``model``: an adapter with an energy tap (``node_energy``), whose engine derivative gives the
    forces. ``evaluate(positions)`` takes float64 host coordinates (any lattice image) and returns
    ``{"e": float, "f": float32 [n, 3]}``. ``capture=False`` runs the same body eagerly."""

    def __init__(self, model, *, atomic_numbers, cell, skin: float = 2.0, capture: bool = True,
                 device: torch.device | str = "cuda", u_step: int = 512, t_step: int = 8192, min_pad_u: int = 256,
                 min_pad_t: int | None = None, warmup: int = 2, check_isolated_atoms: bool = True) -> None:
        if not (np.isfinite(skin) and skin > 0):
            raise ValueError("topology reuse needs a positive skin")
        self.adapter = model
        self._derivative = engine_derivative(model)
        if self._derivative is None:
            raise NotImplementedError("the skin-topology runner differentiates an energy tap (node_energy)")
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.capture = bool(capture)
        self.skin = float(skin)
        self.u_step, self.t_step = int(u_step), int(t_step)
        self.min_pad_u = int(min_pad_u)
        self.min_pad_t = int(self.t_step // 2 if min_pad_t is None else min_pad_t)
        self.warmup = int(warmup)
        self.check_isolated_atoms = bool(check_isolated_atoms)
        self.cell = np.array(cell, dtype=np.float64)
        self._inv_cell = np.linalg.inv(self.cell)
        numbers = torch.as_tensor(np.asarray(atomic_numbers), dtype=torch.int32)
        self.n_real = int(numbers.numel())
        topology = model.topology_spec()
        self.cutoff = float(topology.cutoff)
        self.triplet_cutoff = None if topology.triplet_cutoff is None else float(topology.triplet_cutoff)
        step = model.capacity_step() if hasattr(model, "capacity_step") else None
        self._factors = (1.0, 1.0) if step is None else (float(step.u_thermal_factor), float(step.t_thermal_factor))
        self._builder_args = dict(cell=torch.tensor(self.cell, dtype=torch.float32), atomic_numbers=numbers,
                                  atom_graph_cutoff=self.cutoff, candidate_cutoff=self.cutoff + self.skin,
                                  minimum_image=True, device=self.device, t_capacity=0, line_graph_cutoff=None,
                                  padding=(model.padding_rule() if hasattr(model, "padding_rule")
                                           else PaddingRule("far_self_loops")))
        # the owner holds the candidate list and counts a refresh's exact edge demand (its own
        # capacity is irrelevant: the count covers every row)
        self.owner = FixedCapacityGraphBuilder(u_capacity=1, **self._builder_args)
        self.positions = torch.zeros((self.n_real, 3), dtype=torch.float32, device=self.device)
        self._pinned_positions = torch.empty((self.n_real, 3), dtype=torch.float32, pin_memory=True)
        self._pinned_flags = torch.empty(6, dtype=torch.int64, pin_memory=True)
        self._pinned_energy = torch.empty(1, dtype=torch.float64, pin_memory=True)
        self._pinned_forces = torch.empty((self.n_real, 3), dtype=torch.float32, pin_memory=True)
        self.pool = torch.cuda.graph_pool_handle() if self.capture else None
        self.buckets: dict = {}
        self._reference = None  # host coordinates of the last refresh
        self._demand = None     # (u, t) counts of the last evaluation or refresh
        self.calls = self.refreshes = self.redo_capacity = self.redo_skin = self.captures = 0
        self.max_host_displacement = 0.0
        self.last_edge_count = self.last_triplet_count = 0
        self.last_bucket = None  # (u_cap, t_cap) of the last call's evaluation

    # ------------------------------------------------------------------ buckets
    def _key_for(self, u: int, t: int) -> tuple[int, int]:
        """The bucket of a demand: held above it and tiered (capacity_policy.py:19-24,211-214),
        which leaves at least the minimum padding free."""
        uf, tf = self._factors
        u_cap = tier(held_demand(u, 0, uf), self.u_step, self.min_pad_u)
        if self.triplet_cutoff is None:
            return u_cap, 0
        return u_cap, tier(held_demand(t, 0, tf), self.t_step, self.min_pad_t)

    def _fits(self, key, u: int, t: int) -> bool:
        """Demand (u, t) fits bucket ``key``: an edges-only build holds up to e_cap rows; a
        line-graph build overflows its pairs at e_cap (fixed_capacity_builder.py:796-814)."""
        if self.triplet_cutoff is None:
            return u <= key[0]
        return u < key[0] and t <= key[1]

    def _margin(self, u: int, t: int) -> tuple[int, int]:
        """The demand a bucket is selected for: the last counts plus the minimum padding, so the
        usual call-to-call growth does not overflow (fastmd/execution/skin_topology.py:311-315)."""
        return u + self.min_pad_u, (t + self.min_pad_t if self.triplet_cutoff is not None else 0)

    def _body(self, builder: FixedCapacityGraphBuilder):
        graph, status = builder.build(self.positions, rebuild_candidates=False)
        out = self._derivative(builder.batch, graph, task="ef", n_real=self.n_real)
        flags = torch.cat([status.candidate_valid.reshape(1).long(),
                           builder._candidate_capacity_valid.reshape(1).long(),
                           fixed_capacity_exceeded(status, builder).reshape(1).long(),
                           status.edge_count.reshape(1).long(), status.triplet_count.reshape(1).long(),
                           status.isolated_atom_count.reshape(1).long()])
        return out, flags

    def _make_bucket(self, key) -> dict:
        u_cap, t_cap = key
        kwargs = dict(self._builder_args)
        if self.triplet_cutoff is not None:
            kwargs.update(line_graph_cutoff=self.triplet_cutoff, t_capacity=t_cap)
        builder = FixedCapacityGraphBuilder(u_capacity=u_cap, candidates_from=self.owner,
                                            prepare=self.adapter.prepare, **kwargs)
        entry = {"builder": builder, "graph": None, "out": None, "flags": None}
        if self.capture:
            side = torch.cuda.Stream(device=self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                for _ in range(self.warmup):
                    self._body(builder)
            torch.cuda.current_stream(self.device).wait_stream(side)
            torch.cuda.synchronize(self.device)
            graph = torch.cuda.CUDAGraph()
            with capture_graph(graph, pool=self.pool, name="skin_topology_capture"):
                out, flags = self._body(builder)
            entry.update(graph=graph, out=out, flags=flags)
            self.captures += 1
        self.buckets[key] = entry
        return entry

    def _bucket(self, u: int, t: int) -> dict:
        """The smallest cached bucket that holds the margin over demand (u, t), else a new one."""
        mu, mt = self._margin(u, t)
        fitting = [k for k in self.buckets if self._fits(k, mu, mt)]
        if fitting:
            return self.buckets[min(fitting)]
        return self._make_bucket(self._key_for(mu, mt))

    def close(self) -> None:
        """Release every bucket (graphs and builders) of this system."""
        self.buckets.clear()

    # ------------------------------------------------------------------ evaluation
    def _displacement(self, positions: np.ndarray) -> float:
        """Host minimum-image maximum displacement since the last refresh (A)."""
        delta = positions - self._reference
        delta -= np.rint(delta @ self._inv_cell) @ self.cell
        return float(np.sqrt(np.einsum("ij,ij->i", delta, delta).max(initial=0.0)))

    def _refresh(self, positions: np.ndarray) -> None:
        """New candidates at the runner's device coordinates and their exact edge count (one small
        readback; refreshes are rare and start a call)."""
        self.owner.refresh_candidates(self.positions)
        _, status = self.owner.build(self.positions, rebuild_candidates=False)
        valid, edges = torch.cat([self.owner._candidate_capacity_valid.long(), status.edge_count.long()]).tolist()
        if not valid:
            raise SkinTopologyUnavailable(
                f"a candidate row exceeds {self.owner.buffer_max} slots within {self.owner.candidate_cutoff} A")
        self._reference = np.array(positions, dtype=np.float64, copy=True)
        t = 0 if self._demand is None else self._demand[1]
        self._demand = ((edges + 1) // 2, t)
        self.refreshes += 1

    def _launch(self, entry):
        if entry["graph"] is not None:
            entry["graph"].replay()
            return entry["out"], entry["flags"]
        return self._body(entry["builder"])

    @torch.no_grad()
    def _read(self, out, flags):
        """One readback: the status vector, the float64 energy and the real rows' forces."""
        self._pinned_flags.copy_(flags, non_blocking=True)
        self._pinned_energy.copy_(out["e"].reshape(-1)[:1].to(torch.float64), non_blocking=True)
        self._pinned_forces.copy_(out["f"][0][: self.n_real], non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        return self._pinned_flags.tolist(), {"e": float(self._pinned_energy[0]),
                                             "f": self._pinned_forces.numpy().copy()}

    def evaluate(self, positions) -> dict:
        """Energy (float64) and forces (float32 [n, 3]) at ``positions`` (host, float64, any
        lattice image). Raises ``SkinTopologyUnavailable`` when a candidate row is truncated."""
        with roctx_range("skin_topology_evaluate"), torch.cuda.device(self.device):
            positions = np.asarray(positions, dtype=np.float64)
            if positions.shape != (self.n_real, 3):
                raise ValueError(f"positions must have shape {(self.n_real, 3)}, got {positions.shape}")
            self._pinned_positions.numpy()[...] = positions
            self.positions.copy_(self._pinned_positions, non_blocking=True)
            if self._reference is None:
                self._refresh(positions)
            else:
                moved = self._displacement(positions)
                self.max_host_displacement = max(self.max_host_displacement, moved)
                if moved >= PROACTIVE_REFRESH_FRACTION * self.skin:
                    self._refresh(positions)
            for _ in range(MAX_ATTEMPTS):
                entry = self._bucket(*self._demand)
                flags, result = self._read(*self._launch(entry))
                candidates_valid, capacity_valid, exceeded, edges, triplets, isolated = flags
                if not capacity_valid:
                    raise SkinTopologyUnavailable(f"a candidate row exceeds {self.owner.buffer_max} slots")
                if not candidates_valid:
                    # an atom moved half the skin unseen by the host test: the list is stale
                    self.redo_skin += 1
                    self._refresh(positions)
                    continue
                if exceeded:
                    # the bucket evaluated its padding: redo in one that holds this call's counts
                    builder = entry["builder"]
                    demand = ((edges + 1) // 2, triplets)
                    if self._fits((builder.u_capacity, builder.t_capacity), *demand):
                        raise SkinTopologyUnavailable(f"invalid pair topology at demand {demand}")
                    self._demand = demand
                    self.redo_capacity += 1
                    continue
                break
            else:
                raise RuntimeError(f"skin topology: no valid evaluation in {MAX_ATTEMPTS} attempts")
            self._demand = ((edges + 1) // 2, triplets)
            self.last_edge_count, self.last_triplet_count = edges, triplets
            self.last_bucket = (entry["builder"].u_capacity, entry["builder"].t_capacity)
            self.calls += 1
            if self.check_isolated_atoms and isolated:
                from fastmd_amd.graph.gpu_graph_builder import raise_if_isolated_atoms

                raise_if_isolated_atoms(isolated)
            return result

    def stats(self) -> dict:
        return {"capture": self.capture, "skin": self.skin, "calls": self.calls, "refreshes": self.refreshes,
                "redo_capacity": self.redo_capacity, "redo_skin": self.redo_skin, "captures": self.captures,
                "buckets": sorted(self.buckets), "max_host_displacement": self.max_host_displacement,
                "last_edge_count": self.last_edge_count, "last_triplet_count": self.last_triplet_count,
                "last_bucket": self.last_bucket, "buffer_max": self.owner.buffer_max}
