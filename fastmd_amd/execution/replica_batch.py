"""Replica batching: R independent MD replicas of one system in ONE whole-step graph
(fastmd/execution/replica_batch.py:126-470, whole_step_cuda_graph.py:739-1147).

Small systems leave the GPU idle between launches; R replicas (the same atoms and cell, their own
momenta and thermostat chains) share every launch of the step. The union graph is one
fixed-capacity build over the R·N atoms whose candidate search takes no pair across replicas
(``system_size``), so each replica's rows are its own edge list, in the canonical order, with
the union's atom indices; the model sees one batch, the engine derivative sums one energy per
replica (``EnergyDerivative.segments``), and each replica's NHC chain integrates its own rows.
A replica's trajectory is therefore bitwise the single-system run with its momenta (tested)
while the union's node GEMMs take the form the single system's take (fp32 tiles below a
launch-size threshold, about 4 000 rows for the MACE-like model; above it the split-plane form,
and the replicas match their single runs to float32 rounding).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from fastmd_amd import units
from fastmd_amd.config import InferenceConfig
from fastmd_amd.engine.capacity_policy import JointCapacityPolicy, held_demand, whole_step_headroom
from fastmd_amd.execution.cuda_graph import triplet_demand
from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT, NHCState, maxwell_boltzmann_momenta
from fastmd_amd.execution.whole_step_cuda_graph import FixedCapacityOverflow, WholeStepGraphRunner
from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder
from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder


@dataclass
class ReplicaNHCState:
    """Views into one flat float64 buffer: the union rows (replica r: rows [r N, (r+1) N)) and the
    per-replica chains and energies (replica_batch.py:282-312)."""

    flat: Tensor
    positions: Tensor  # [R N, 3]
    momenta: Tensor
    forces: Tensor
    eta: Tensor  # [R, tchain]
    p_eta: Tensor
    potential_energy: Tensor  # [R]

    @staticmethod
    def allocate(replicas: int, n_atoms: int, tchain: int, device) -> "ReplicaNHCState":
        rows = 3 * replicas * n_atoms
        flat = torch.zeros(3 * rows + 2 * replicas * tchain + replicas, dtype=torch.float64, device=device)
        o = 0
        views = []
        for size, shape in ((rows, (replicas * n_atoms, 3)), (rows, (replicas * n_atoms, 3)),
                            (rows, (replicas * n_atoms, 3)), (replicas * tchain, (replicas, tchain)),
                            (replicas * tchain, (replicas, tchain)), (replicas, (replicas,))):
            views.append(flat[o:o + size].view(*shape))
            o += size
        return ReplicaNHCState(flat, *views)

    def replica(self, r: int, n: int) -> NHCState:
        s = slice(r * n, (r + 1) * n)
        return NHCState(None, self.positions[s], self.momenta[s], self.forces[s], self.eta[r], self.p_eta[r],
                        self.potential_energy[r:r + 1])


class ReplicaNoseHooverChainNVT:
    """R Nose-Hoover chains (ASE-exact, one ``GPUNoseHooverChainNVT`` each, the same kernels) over
    one union state; the whole-step runner's integrator protocol on the union rows
    (replica_batch.py:314-470)."""

    ensemble = "nvt_nhc"

    def __init__(self, masses, positions, momenta, *, replicas: int, temperature_K: float, timestep: float,
                 tdamp: float, tchain: int = 3, tloop: int = 1, device="cuda",
                 force_dtype: torch.dtype = torch.float32) -> None:
        self.replicas = int(replicas)
        if self.replicas < 1:
            raise ValueError("replicas must be >= 1")
        masses = np.asarray(masses, np.float64).reshape(-1)
        n = self.n_replica_atoms = int(masses.shape[0])
        self.n_atoms = self.replicas * n
        self.tchain = int(tchain)
        self.device = torch.device(device)
        positions = np.array(np.broadcast_to(np.asarray(positions, np.float64).reshape(-1, n, 3), (self.replicas, n, 3)))
        momenta = np.asarray(momenta, np.float64).reshape(self.replicas, n, 3)
        self.state = ReplicaNHCState.allocate(self.replicas, n, self.tchain, self.device)
        self._backup = ReplicaNHCState.allocate(self.replicas, n, self.tchain, self.device)
        self._subs = []
        for r in range(self.replicas):
            sub = GPUNoseHooverChainNVT(masses, positions[r], momenta[r], temperature_K=temperature_K,
                                        timestep=timestep, tdamp=tdamp, tchain=tchain, tloop=tloop, device=device,
                                        force_dtype=force_dtype)
            view = self.state.replica(r, n)
            for name in ("positions", "momenta", "forces", "eta", "p_eta", "potential_energy"):
                getattr(view, name).copy_(getattr(sub.state, name))
            sub.state = view  # the chain integrates its rows of the union state
            self._subs.append(sub)
        self.masses = self._subs[0].masses

    @property
    def temperature_K(self) -> float:
        return self._subs[0].temperature_K

    def set_temperature(self, temperature_K: float) -> None:
        for sub in self._subs:
            sub.set_temperature(temperature_K)

    # the union rows
    @property
    def positions(self) -> Tensor:
        return self.state.positions

    @property
    def momenta(self) -> Tensor:
        return self.state.momenta

    @property
    def forces(self) -> Tensor:
        return self.state.forces

    @property
    def potential_energy(self) -> Tensor:
        return self.state.potential_energy

    @property
    def eta(self) -> Tensor:
        return self.state.eta

    @property
    def p_eta(self) -> Tensor:
        return self.state.p_eta

    def replica(self, r: int) -> GPUNoseHooverChainNVT:
        return self._subs[r]

    @torch.no_grad()
    def set_state(self, *, positions=None, momenta=None, forces=None, potential_energy=None) -> None:
        st = self.state
        for name, value in (("positions", positions), ("momenta", momenta), ("forces", forces)):
            if value is not None:
                getattr(st, name).copy_(torch.as_tensor(value, dtype=torch.float64, device=self.device)
                                        .reshape(self.n_atoms, 3))
        if potential_energy is not None:
            st.potential_energy.copy_(torch.as_tensor(potential_energy, dtype=torch.float64,
                                                      device=self.device).reshape(self.replicas))

    def set_forces(self, forces, energy=None) -> None:
        self.state.forces.copy_(forces.reshape(self.n_atoms, 3))
        if energy is not None:
            self.state.potential_energy.copy_(energy.reshape(self.replicas).to(torch.float64))

    def step_pre_force(self) -> Tensor:
        for sub in self._subs:
            sub.step_pre_force()
        return self.state.positions

    def step_post_force(self, forces: Tensor, energy: Tensor | None = None) -> None:
        n = self.n_replica_atoms
        forces = forces.reshape(self.n_atoms, 3)
        energy = None if energy is None else energy.reshape(-1)
        if energy is not None and energy.numel() != self.replicas:
            raise ValueError(f"one energy per replica expected, got {energy.numel()}")
        for r, sub in enumerate(self._subs):
            sub.step_post_force(forces[r * n:(r + 1) * n], energy=None if energy is None else energy[r:r + 1])

    # transactions on the union state
    def backup(self, state: ReplicaNHCState | None = None) -> None:
        self._backup.flat.copy_((self.state if state is None else state).flat)

    def restore(self, state: ReplicaNHCState | None = None) -> None:
        (self.state if state is None else state).flat.copy_(self._backup.flat)

    def snapshot(self) -> tuple:
        return self.state.flat.clone(), self._backup.flat.clone()

    def load_snapshot(self, snapshot: tuple) -> None:
        state, backup = snapshot
        self.state.flat.copy_(state)
        self._backup.flat.copy_(backup)

    def new_state(self) -> ReplicaNHCState:
        return ReplicaNHCState.allocate(self.replicas, self.n_replica_atoms, self.tchain, self.device)

    # observables per replica
    def kinetic_energy(self) -> Tensor:
        return torch.stack([sub.kinetic_energy() for sub in self._subs])

    def temperature(self) -> Tensor:
        return torch.stack([sub.temperature() for sub in self._subs])

    def conserved_energy(self) -> Tensor:
        return torch.stack([sub.conserved_energy() for sub in self._subs])


class ReplicaBatchedMD:
    """R replicas of one system (their own momenta and thermostats) in one whole-step graph
    per window: ``GPUResidentMolecularDynamics``'s parameters plus ``replicas`` and per-replica
    ``seeds`` or ``momenta`` [R, N, 3]; ``run(steps)``, per-replica ``thermodynamics()``."""

    def __init__(self, atoms, model, *, replicas: int, device: torch.device | str = "cuda",
                 temperature: float = 300.0, timestep: float = 1.0, tdamp: float = 100.0, tchain: int = 3,
                 tloop: int = 1, seeds=None, momenta=None, steps_per_launch: int = 1,
                 config: InferenceConfig | None = None, validate_isolated_atoms: bool = False) -> None:
        from fastmd_amd.interfaces.gpu_md import _atoms_arrays

        self.config = config or InferenceConfig()
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.adapter = model
        self.replicas = int(replicas)
        self.steps_per_launch = int(steps_per_launch)
        self.validate_isolated_atoms = bool(validate_isolated_atoms)
        positions, cell, numbers, masses, _ = _atoms_arrays(atoms)
        n = self.n_atoms = int(positions.shape[0])
        if momenta is None:
            seeds = list(range(self.replicas)) if seeds is None else list(seeds)
            if len(seeds) != self.replicas:
                raise ValueError("one seed per replica")
            momenta = np.stack([maxwell_boltzmann_momenta(masses, temperature, s) for s in seeds])
        momenta = np.asarray(momenta, np.float64).reshape(self.replicas, n, 3)
        self.timestep_fs = float(timestep)
        self.integrator = ReplicaNoseHooverChainNVT(
            masses, positions, momenta, replicas=self.replicas, temperature_K=temperature,
            timestep=timestep * units.fs, tdamp=tdamp * units.fs, tchain=tchain, tloop=tloop, device=self.device)
        self.cell = torch.tensor(cell, dtype=torch.float64)
        self.numbers = torch.tensor(np.tile(np.asarray(numbers), self.replicas), dtype=torch.int32)
        topology = model.topology_spec()
        self.cutoff = float(topology.cutoff)
        self.triplet_cutoff = None if topology.triplet_cutoff is None else float(topology.triplet_cutoff)
        # demand: R times one replica's ragged build
        single = TensorGraphBuilder(cell=self.cell, atomic_numbers=torch.tensor(numbers, dtype=torch.int32),
                                    atom_graph_cutoff=self.cutoff, line_graph_cutoff=None, device=self.device,
                                    check_isolated_atoms=False)
        sample = single.build(torch.as_tensor(positions, dtype=torch.float64, device=self.device))
        u = self.replicas * (int(sample.edge_index.shape[0]) // 2)
        t = self.replicas * triplet_demand(sample, self.triplet_cutoff) if self.triplet_cutoff is not None else 0
        step = model.capacity_step() if hasattr(model, "capacity_step") else None
        cap = self.config.capacity
        self._u_step, self._min_pad = (step.u_step, step.min_pad_u) if step is not None else (cap.u_step, cap.min_pad_u)
        self._factors = (step.u_thermal_factor, step.t_thermal_factor) if step is not None else (1.0, 1.0)
        t_step = (step.t_step or 128) if step is not None else cap.t_step
        self.policy = JointCapacityPolicy(u_step=self._u_step, min_pad_u=self._min_pad,
                                          t_step=t_step if self.triplet_cutoff is not None else None,
                                          min_pad_t=(step.min_pad_t if step is not None else cap.min_pad_t))
        self._t_step = t_step
        self._capacity = self.policy.start(*self._held(u, t))
        self._pool = torch.cuda.graph_pool_handle()
        self.steps = 0
        self.runner = None
        self.capacity_history = []
        self._make_runner(recapture=False)

    def _held(self, u: int, t: int) -> tuple[int, int]:
        uf, tf = self._factors
        hu = held_demand(u, whole_step_headroom(u, self._u_step), uf)
        ht = held_demand(t, whole_step_headroom(t, self._t_step), tf) if self.triplet_cutoff is not None else 0
        return hu, ht

    def _make_runner(self, recapture: bool) -> None:
        while True:
            key = self._capacity
            builder = FixedCapacityGraphBuilder(
                cell=self.cell, atomic_numbers=self.numbers, u_capacity=key.u_capacity,
                t_capacity=key.t_capacity if self.triplet_cutoff is not None else 0, atom_graph_cutoff=self.cutoff,
                line_graph_cutoff=self.triplet_cutoff, candidate_cutoff=self.cutoff + self.config.capacity.candidate_skin,
                padding=self.adapter.padding_rule(), prepare=self.adapter.prepare, device=self.device,
                system_size=self.n_atoms)
            try:
                self.runner = WholeStepGraphRunner(model=self.adapter, builder=builder, integrator=self.integrator,
                                                   steps_per_launch=self.steps_per_launch,
                                                   warmup=self.config.capacity.warmup, graph_pool=self._pool,
                                                   validate_isolated_atoms=self.validate_isolated_atoms,
                                                   recapture=recapture)
                self.capacity_history.append((key.u_capacity, key.t_capacity))
                return
            except FixedCapacityOverflow as overflow:
                self._grow(overflow)

    def _grow(self, overflow: FixedCapacityOverflow) -> None:
        self._capacity = self.policy.grow(self._capacity, *self._held((overflow.edge_count + 1) // 2,
                                                                      overflow.triplet_count))

    def run(self, steps: int) -> None:
        """``steps`` MD steps of every replica (a multiple of ``steps_per_launch``)."""
        if steps % self.steps_per_launch:
            raise ValueError(f"steps ({steps}) must be a multiple of steps_per_launch ({self.steps_per_launch})")
        done = 0
        while done < steps:
            try:
                self.runner.replay()
            except FixedCapacityOverflow as overflow:
                self._grow(overflow)
                self.runner = None
                self._make_runner(recapture=True)
                continue
            done += self.steps_per_launch
            self.steps += self.steps_per_launch

    def replica_state(self, r: int) -> dict:
        """Views of replica r's positions, momenta and forces (float64 [N, 3]) and its energy."""
        n = self.n_atoms
        s = slice(r * n, (r + 1) * n)
        st = self.integrator.state
        return {"positions": st.positions[s], "momenta": st.momenta[s], "forces": st.forces[s],
                "potential_energy": st.potential_energy[r]}

    def thermodynamics(self) -> list[dict]:
        """Per replica: step, potential / kinetic / total energy, temperature, conserved energy."""
        th = self.integrator
        epot = th.potential_energy.tolist()
        ekin = th.kinetic_energy().tolist()
        temp = th.temperature().tolist()
        cons = th.conserved_energy().tolist()
        return [{"step": self.steps, "time_fs": self.steps * self.timestep_fs, "potential_energy": epot[r],
                 "kinetic_energy": ekin[r], "total_energy": epot[r] + ekin[r], "temperature": temp[r],
                 "conserved_energy": cons[r]} for r in range(self.replicas)]

    def stats(self) -> dict:
        st = self.runner.stats()
        st["capacity_history"] = list(self.capacity_history)
        return st
