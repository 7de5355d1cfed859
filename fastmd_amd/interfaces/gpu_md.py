"""GPU-resident molecular dynamics on one MI355X: the drop-in driver of the MD step.

Interface of the reference's ``GPUResidentMolecularDynamics`` (fastmd/interfaces/gpu_md.py:
135-462 constructor, ``step`` :1789-1830, ``run`` :1866-1880, ``evaluate`` :1500-1529,
``conserved_energy`` :1999-2004, ``thermodynamics`` :2169-2204, ``whole_step_stats`` :2007) for
the Nose-Hoover chain ensemble and an energy-tap model adapter. ``atoms`` is an ASE-like object
(``get_positions``/``get_cell``/``get_atomic_numbers``/``get_masses`` and optionally
``get_momenta``) or a ``fastmd_amd.systems.System``; ASE itself is not a dependency.

Execution modes (``InferenceConfig.execution``):
  ``eager``       per step: ragged exact neighbour list (host syncs) -> model -> NHC halves;
  ``model_graph`` per step: ragged build -> the model's forward + VJP replayed as the hipGraph of
                  the capacity bucket that holds it (``execution.cuda_graph.BucketedGraphRunner``)
                  -> NHC halves (gpu_md.py:435-446, 560-590);
  ``whole_step``  the whole step captured as one hipGraph per capacity tier, replayed per
                  window of ``steps_per_launch`` steps (``auto`` selects it).
Units: ``timestep``, ``tdamp`` in fs, ``temperature`` in K (ASE units inside).
"""
from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from fastmd_amd import units
from fastmd_amd.config import InferenceConfig
from fastmd_amd.engine.capacity_policy import JointCapacityPolicy, held_demand, whole_step_headroom
from fastmd_amd.engine.energy_derivative import engine_derivative
from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT, maxwell_boltzmann_momenta
from fastmd_amd.execution.whole_step_cuda_graph import (FixedCapacityOverflow, WholeStepGraphRunner,
                                                        _capacity_exceeded)
from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder
from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder, raise_if_isolated_atoms


def _atoms_arrays(atoms):
    if hasattr(atoms, "get_positions"):
        positions = np.asarray(atoms.get_positions(), dtype=np.float64)
        cell = np.asarray(getattr(atoms.get_cell(), "array", atoms.get_cell()), dtype=np.float64)
        numbers = np.asarray(atoms.get_atomic_numbers(), dtype=np.int32)
        masses = np.asarray(atoms.get_masses(), dtype=np.float64)
        momenta = np.asarray(atoms.get_momenta(), dtype=np.float64) if hasattr(atoms, "get_momenta") else None
        if momenta is not None and not np.any(momenta):
            momenta = None
        return positions, cell, numbers, masses, momenta
    return (np.asarray(atoms.positions, dtype=np.float64), np.asarray(atoms.cell, dtype=np.float64),
            np.asarray(atoms.numbers, dtype=np.int32), np.asarray(atoms.masses, dtype=np.float64),
            getattr(atoms, "momenta", None))


# runner counters summed over the runners a capacity growth retires (whole_step_stats covers the run)
_CUMULATIVE_STATS = ("launches", "candidate_refreshes", "fallback_windows", "recovery_replays", "warmup_runs")


class GPUResidentMolecularDynamics:
    def __init__(self, atoms, model=None, *, device: torch.device | str = "cuda", ensemble: str = "nvt_nhc",
                 temperature: float = 300.0, timestep: float = 1.0, taut: float = 100.0, tdamp: float | None = None,
                 tchain: int = 3, tloop: int = 1, config: InferenceConfig | None = None, steps_per_launch: int = 1,
                 momenta=None, seed: int = 0, task: str = "ef", validate_isolated_atoms: bool = False) -> None:
        if ensemble.lower() != "nvt_nhc":
            raise NotImplementedError("this build integrates the Nose-Hoover chain ensemble (ensemble='nvt_nhc')")
        if model is None or not hasattr(model, "node_energy"):
            raise TypeError("model must be a model adapter with an energy tap (node_energy)")
        if isinstance(steps_per_launch, bool) or not isinstance(steps_per_launch, int) or steps_per_launch < 1:
            raise ValueError("GPUResidentMolecularDynamics: steps_per_launch must be a positive integer")
        self.config = config or InferenceConfig()
        self.execution = self.config.resolved_execution
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.adapter = model
        self.derivative = engine_derivative(model)
        self.task = task
        self.steps_per_launch = int(steps_per_launch)
        # run(): launch each next whole-step window before the host reads the flags of the one in
        # flight (see run); counters of the windows launched so and of those rolled back
        self.launch_behind = True
        self.windows_ahead = 0
        self.windows_rolled_back = 0
        self.validate_isolated_atoms = bool(validate_isolated_atoms)
        positions, cell, numbers, masses, atom_momenta = _atoms_arrays(atoms)
        self.n_atoms = int(positions.shape[0])
        self.cell = torch.tensor(cell, dtype=torch.float64)
        self.numbers = torch.tensor(numbers, dtype=torch.int32)
        self.masses = masses
        self.temperature = float(temperature)
        if momenta is None:
            momenta = atom_momenta if atom_momenta is not None else maxwell_boltzmann_momenta(masses, temperature, seed)
        tdamp = taut if tdamp is None else tdamp
        self.integrator = GPUNoseHooverChainNVT(
            masses, positions, np.asarray(momenta, dtype=np.float64), temperature_K=temperature,
            timestep=timestep * units.fs, tdamp=tdamp * units.fs, tchain=tchain, tloop=tloop, device=self.device,
            force_dtype=torch.float32)
        topology = model.topology_spec()
        self.cutoff = float(topology.cutoff)
        # a three-body model reads the line graph of bonds shorter than this (None: edges only)
        self.triplet_cutoff = None if topology.triplet_cutoff is None else float(topology.triplet_cutoff)
        self.graph_builder = TensorGraphBuilder(cell=self.cell, atomic_numbers=self.numbers,
                                                atom_graph_cutoff=self.cutoff, device=self.device,
                                                check_isolated_atoms=False)
        self._eager_line = None  # the eager path's line-graph builder and its capacity
        self.model_runner = None  # model_graph: the bucketed model graphs
        self.steps = 0
        self.whole_step_runner: WholeStepGraphRunner | None = None
        self.capacity_policy = None
        self._capacity = None
        self.whole_step_capacity_history: list[int] = []
        self.whole_step_triplet_capacity_history: list[int] = []
        self._retired_stats: dict = {}
        self._graph_pool = None
        if self.execution == "model_graph":
            self.enable_model_cuda_graph()
        # F(q0) for the first pre-force half
        forces, energy = self.evaluate(self.integrator.positions)
        self.integrator.set_forces(forces, energy=energy)
        if self.execution == "whole_step":
            self.enable_whole_step_cuda_graph()

    # ------------------------------------------------------------------ eager evaluation
    def evaluate(self, positions: Tensor | None = None) -> tuple[Tensor, Tensor]:
        """(forces float32 [N, 3], energy float64 [1]) at ``positions`` (default: the current
        state), through a ragged exact neighbour list (eager, host syncs); in the model_graph
        mode by the replay of the bucket's model graph (copies: the graph's outputs are reused)."""
        forces, energy = self._evaluate(positions)
        if self.model_runner is not None:
            return forces.clone(), energy.clone()
        return forces, energy

    def _evaluate(self, positions: Tensor | None = None) -> tuple[Tensor, Tensor]:
        q = self.integrator.positions if positions is None else positions
        if self.model_runner is not None:
            batch = self.graph_builder.build(q)
            if self.validate_isolated_atoms:
                counts = torch.diff(batch.edge_offsets)
                raise_if_isolated_atoms(int((counts == 0).sum().item()))
            out, n = self.model_runner.run(batch, positions=q)
            return out["f"][0][:n].detach(), out["e"].detach()
        batch = self._eager_batch(q)
        if self.validate_isolated_atoms:
            counts = torch.diff(batch.edge_offsets)
            raise_if_isolated_atoms(int((counts == 0).sum().item()))
        inputs = self.adapter.prepare(batch)
        out = self.derivative(batch, inputs, task=self.task, n_real=self.n_atoms)
        return out["f"][0][: self.n_atoms].detach(), out["e"].detach()

    def enable_model_cuda_graph(self) -> None:
        """The model_graph mode (gpu_md.py:560-590): the model's forward + VJP as one graph per
        capacity bucket, the ragged build and the integrator eager."""
        if self.whole_step_runner is not None:
            raise ValueError("cannot enable model replay with a whole-step runner")
        if self.model_runner is not None:
            return
        from fastmd_amd.execution.cuda_graph import BucketedGraphRunner

        cap = self.config.capacity
        u_step, min_pad, _ = self._capacity_step()
        t_step, t_pad, _ = self._triplet_step() if self.triplet_cutoff is not None else (cap.t_step, cap.min_pad_t, 1.0)
        self.model_runner = BucketedGraphRunner(self.adapter, task=self.task, u_step=u_step, t_step=t_step,
                                                n_dummy=cap.n_dummy, min_pad_u=min_pad, warmup=cap.warmup,
                                                min_pad_t=t_pad, candidate_skin=cap.candidate_skin, device=self.device)

    def model_graph_stats(self) -> dict:
        if self.model_runner is None:
            raise RuntimeError("the model_graph mode is not enabled")
        return self.model_runner.stats()

    def step(self) -> None:
        """One eager MD step (integrator halves around a fresh evaluation)."""
        if self.whole_step_runner is not None:
            raise RuntimeError("step() is the eager path; the whole-step mode runs windows through run()")
        q = self.integrator.step_pre_force()
        forces, energy = self._evaluate(q)
        self.integrator.step_post_force(forces, energy=energy)
        self.steps += 1

    def _demand(self, batch) -> tuple[int, int]:
        """(undirected pairs, triplets) of a ragged build: the pairs from its edge count, the
        triplets from its bonds (squared float32 length below the bond cutoff's, the builder's
        own test) as sum s (s - 1) over the centres."""
        u = int(batch.edge_index.shape[0]) // 2
        if self.triplet_cutoff is None:
            return u, 0
        ei = batch.edge_index.long()
        cell = batch.cell.to(torch.float32)
        pos = batch.positions.to(torch.float32)
        vec = pos.index_select(0, ei[:, 1]) + batch.edge_image.to(torch.float32) @ cell - pos.index_select(0, ei[:, 0])
        short = (vec * vec).sum(1) < float(np.float32(self.triplet_cutoff * self.triplet_cutoff))
        s = torch.bincount(ei[short, 0], minlength=self.n_atoms)
        return u, int((s * (s - 1)).sum().item())

    def _eager_batch(self, q: Tensor):
        """The batch of an eager evaluation: the ragged exact list, or for a three-body model a
        line-graph build at a capacity held above the ragged list's demand (regrown when short)."""
        batch = self.graph_builder.build(q)
        if self.triplet_cutoff is None:
            return batch
        u, t = self._demand(batch)
        policy = self._policy()
        want = policy.key_for(*self._held(u, t))
        while True:
            if self._eager_line is None or (self._eager_line[1].u_capacity < want.u_capacity
                                            or self._eager_line[1].t_capacity < want.t_capacity):
                key = want if self._eager_line is None else policy.grow(self._eager_line[1], *self._held(u, t))
                self._eager_line = (self._line_builder(key, prepare=None), key)
            builder = self._eager_line[0]
            builder.refresh_candidates(q)
            _, status = builder.build(q, rebuild_candidates=False)
            if not _capacity_exceeded(builder, status):
                return builder.batch
            u = max(u, (int(status.edge_count.item()) + 1) // 2)
            t = max(t, int(status.triplet_count.item()))
            want = policy.grow(self._eager_line[1], *self._held(u, t))

    # ------------------------------------------------------------------ whole step
    def _line_builder(self, key, prepare):
        return FixedCapacityGraphBuilder(cell=self.cell, atomic_numbers=self.numbers, u_capacity=key.u_capacity,
                                         t_capacity=key.t_capacity if self.triplet_cutoff is not None else 0,
                                         atom_graph_cutoff=self.cutoff, line_graph_cutoff=self.triplet_cutoff,
                                         candidate_cutoff=self.cutoff + self.config.capacity.candidate_skin,
                                         padding=self.adapter.padding_rule(), prepare=prepare, device=self.device)

    def _make_runner(self, key, recapture: bool) -> WholeStepGraphRunner:
        builder = self._line_builder(key, prepare=self.adapter.prepare)
        return WholeStepGraphRunner(model=self.adapter, builder=builder, integrator=self.integrator, task=self.task,
                                    steps_per_launch=self.steps_per_launch, warmup=self.config.capacity.warmup,
                                    graph_pool=self._graph_pool, validate_isolated_atoms=self.validate_isolated_atoms,
                                    recapture=recapture)

    def _capacity_step(self):
        cap = self.config.capacity
        step = getattr(self.adapter, "capacity_step", None)
        if step is not None and (cap.u_step, cap.min_pad_u) == (512, 256):
            s = step()
            return s.u_step, s.min_pad_u, s.u_thermal_factor
        return cap.u_step, cap.min_pad_u, 1.0

    def _triplet_step(self):
        """(t_step, min_pad_t, t_factor): the model's triplet tiers, else 128 / 128 / 1.06."""
        step = getattr(self.adapter, "capacity_step", None)
        s = step() if step is not None else None
        if s is None or not s.t_step:
            return 128, 128, 1.06
        return int(s.t_step), int(s.min_pad_t or s.t_step), float(s.t_thermal_factor)

    def _policy(self) -> JointCapacityPolicy:
        if self.capacity_policy is None:
            u_step, min_pad, _ = self._capacity_step()
            t_step, t_pad, _ = self._triplet_step() if self.triplet_cutoff is not None else (None, None, 1.0)
            self.capacity_policy = JointCapacityPolicy(u_step=u_step, min_pad_u=min_pad, t_step=t_step, min_pad_t=t_pad)
        return self.capacity_policy

    def _held(self, u: int, t: int) -> tuple[int, int]:
        """The pair and triplet counts a capture holds for a demand (headroom, thermal factors)."""
        u_step, _, factor = self._capacity_step()
        held_u = held_demand(u, whole_step_headroom(u, u_step), factor)
        if self.triplet_cutoff is None:
            return held_u, 0
        t_step, _, t_factor = self._triplet_step()
        return held_u, held_demand(t, whole_step_headroom(t, t_step), t_factor)

    def enable_whole_step_cuda_graph(self) -> None:
        """Size the capacity from a ragged build (gpu_md.py:591-711) and capture the window."""
        if self.whole_step_runner is not None:
            return
        sample = self.graph_builder.build(self.integrator.positions)
        u, t = self._demand(sample)
        self._capacity = self._policy().start(*self._held(u, t))
        self._graph_pool = torch.cuda.graph_pool_handle()
        while True:
            try:
                self.whole_step_runner = self._make_runner(self._capacity, recapture=False)
                break
            except FixedCapacityOverflow as overflow:
                self._grow(overflow.edge_count, overflow.triplet_count)
        self.whole_step_capacity_history.append(self._capacity.u_capacity)
        self.whole_step_triplet_capacity_history.append(self._capacity.t_capacity)

    def _grow(self, edge_count: int, triplet_count: int = 0) -> None:
        """A larger tier for a window's largest counts (a pair overflow truncates the triplets it
        counted: their tier grows again if the next window still overflows)."""
        u = (int(edge_count) + 1) // 2
        self._capacity = self._policy().grow(self._capacity, *self._held(u, int(triplet_count)))

    def _grow_whole_step_runner(self, edge_count: int, triplet_count: int = 0) -> None:
        """Capacity growth after an overflowed window: a larger tier, recaptured (gpu_md.py:1355-1410)."""
        old = self.whole_step_runner
        # the retired runner's counters carry over into whole_step_stats()
        for key, value in old.stats().items():
            if key in _CUMULATIVE_STATS:
                self._retired_stats[key] = self._retired_stats.get(key, 0) + value
        self._retired_stats["max_edge_count"] = max(self._retired_stats.get("max_edge_count", 0),
                                                    old.stats()["max_edge_count"])
        self._grow(edge_count, triplet_count)
        self.whole_step_runner = None
        del old
        self.whole_step_runner = self._make_runner(self._capacity, recapture=True)
        self.whole_step_capacity_history.append(self._capacity.u_capacity)
        self.whole_step_triplet_capacity_history.append(self._capacity.t_capacity)

    def run(self, steps: int) -> None:
        """``steps`` MD steps (a multiple of ``steps_per_launch`` in the whole-step mode).

        Whole-step windows are pipelined as the reference's ``_run_windows``
        (gpu_md.py:1882-1975): the next window is launched before the host reads the flags of the
        one in flight, unless that one will likely refresh the candidates, so the GPU does not wait
        for the host (graph submission, flag read) between windows. When the settled window needs
        more than bookkeeping, the window behind it is rolled back: to the settled window's end
        before a candidate refresh, to its start before a fallback or a capacity growth; the
        trajectory is the one of windows settled one at a time, bitwise."""
        steps = int(steps)
        if self.whole_step_runner is None:
            for _ in range(steps):
                self.step()
            return
        if steps % self.steps_per_launch:
            raise ValueError(f"steps ({steps}) must be a multiple of steps_per_launch ({self.steps_per_launch})")
        windows = steps // self.steps_per_launch
        done = 0
        ahead = None  # the slot of the window launched behind the one being settled
        runner = None
        try:
            while done < windows:
                runner = self.whole_step_runner
                slot, ahead = (runner.launch() if ahead is None else ahead), None
                # the next window goes into the stream before the host reads this one's flags (so the
                # GPU does not wait for the host between windows), unless this one will likely
                # refresh the candidates (gpu_md.py:1882-1975)
                if self.launch_behind and done + 1 < windows and runner.refresh_unlikely():
                    ahead = runner.launch(behind=True)
                    self.windows_ahead += 1
                stats = runner.launched_stats(slot)
                work = runner.settling_work(stats)
                if ahead is not None and work is not None:
                    # the window behind ran on what this one's settling changes: roll it back (to this
                    # window's end for a candidate refresh, to this window's start for a fallback or
                    # a growth) and settle this one as if nothing had been launched behind it
                    if work == "refresh":
                        runner.drop()
                    else:
                        runner.rewind()
                    ahead = None
                    self.windows_rolled_back += 1
                try:
                    runner.settle(stats)
                except FixedCapacityOverflow as overflow:
                    self._grow_whole_step_runner(overflow.edge_count, overflow.triplet_count)
                    continue
                done += 1
                self.steps += self.steps_per_launch
        except BaseException:
            if ahead is not None:  # back to the end of the window settled (or being settled)
                runner.drop()
            raise

    # ------------------------------------------------------------------ observables
    @property
    def positions(self) -> Tensor:
        return self.integrator.positions

    @property
    def momenta(self) -> Tensor:
        return self.integrator.momenta

    @property
    def forces(self) -> Tensor:
        return self.integrator.forces

    def conserved_energy(self) -> float:
        return float(self.integrator.conserved_energy())

    def thermodynamics(self) -> dict:
        """One download of the scalars (gpu_md.py:2169-2204)."""
        epot = self.integrator.potential_energy[0]
        ekin = self.integrator.kinetic_energy()
        values = torch.stack([epot, ekin, self.integrator.temperature(), self.integrator.conserved_energy()]).tolist()
        return {"step": self.steps, "epot": values[0], "ekin": values[1], "temperature": values[2],
                "etotal": values[0] + values[1], "conserved": values[3]}

    def whole_step_stats(self) -> dict | None:
        if self.whole_step_runner is None:
            return None
        stats = self.whole_step_runner.stats()
        for key in _CUMULATIVE_STATS:
            stats[key] += self._retired_stats.get(key, 0)
        stats["max_edge_count"] = max(stats["max_edge_count"], self._retired_stats.get("max_edge_count", 0))
        stats["capacity_history"] = list(self.whole_step_capacity_history)
        if self.triplet_cutoff is not None:
            stats["triplet_capacity_history"] = list(self.whole_step_triplet_capacity_history)
        stats["windows_ahead"] = self.windows_ahead
        stats["windows_rolled_back"] = self.windows_rolled_back
        return stats
