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
from fastmd_amd._roctx import roctx_ranged


def _is_out_of_memory(error: BaseException) -> bool:
    """A device allocation failure (torch's, or the HIP runtime's reported as a RuntimeError)."""
    if isinstance(error, torch.OutOfMemoryError):
        return True
    text = str(error).lower()
    return isinstance(error, RuntimeError) and ("out of memory" in text or "hiperroroutofmemory" in text)


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
                 momenta=None, seed: int = 0, task: str = "ef", validate_isolated_atoms: bool = False,
                 trajectory=None, logfile=None, loginterval: int = 1, append_trajectory: bool = False,
                 logger_ring: int = 8, output_dir=None, thermo_interval: int = 0, xyz_interval: int = 0,
                 restart_interval: int = 0, total_steps: int | None = None, restart=None) -> None:
        intervals = (thermo_interval, xyz_interval, restart_interval, 0 if total_steps is None else total_steps)
        if any(isinstance(v, bool) or not isinstance(v, int) or v < 0 for v in intervals):
            raise ValueError("GPUResidentMolecularDynamics: output intervals and total_steps must be nonnegative "
                             "integers")
        if steps_per_launch > 1 if isinstance(steps_per_launch, int) else False:
            # every output and log step must end a window (gpu_md.py:183-195)
            logs = trajectory is not None or logfile is not None
            cadence = {"loginterval": max(int(loginterval), 1) if logs else 0, "thermo_interval": thermo_interval,
                       "xyz_interval": xyz_interval, "restart_interval": restart_interval,
                       "total_steps": total_steps or 0, "restart step": 0 if restart is None else int(restart.step)}
            off = {k: v for k, v in cadence.items() if v % steps_per_launch}
            if off:
                raise ValueError(f"GPUResidentMolecularDynamics: steps_per_launch={steps_per_launch} must divide "
                                 f"{off} (a multi-step window's inner steps are not visible)")
        if ensemble.lower() != "nvt_nhc":
            raise NotImplementedError("this build integrates the Nose-Hoover chain ensemble (ensemble='nvt_nhc')")
        if model is None or not hasattr(model, "node_energy"):
            raise TypeError("model must be a model adapter with an energy tap (node_energy)")
        if isinstance(steps_per_launch, bool) or not isinstance(steps_per_launch, int) or steps_per_launch < 1:
            raise ValueError("GPUResidentMolecularDynamics: steps_per_launch must be a positive integer")
        self.config = config or InferenceConfig()
        self.execution = self.config.resolved_execution
        # execution="auto": an out-of-memory error in a whole-step capture (construction or a
        # capacity growth) continues on the eager path (gpu_md.py:1720-1774); the reason is kept
        self.auto = self.config.execution in (None, "auto")
        self.auto_reason = None
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
        # per-atom masses given explicitly (a System, or ASE atoms holding a masses array): frames
        # then carry a masses column, as ASE's EXTXYZ writer does for such atoms
        self.explicit_masses = not hasattr(atoms, "get_positions") or "masses" in getattr(atoms, "arrays", {})
        self.temperature = float(temperature)
        if momenta is None:
            momenta = atom_momenta if atom_momenta is not None else maxwell_boltzmann_momenta(masses, temperature, seed)
        tdamp = taut if tdamp is None else tdamp
        self.timestep_fs = float(timestep)
        self.parameters = {"ensemble": "nvt_nhc", "temperature_K": float(temperature), "timestep_fs": float(timestep),
                           "tdamp_fs": float(tdamp), "tchain": int(tchain), "tloop": int(tloop),
                           "total_steps": total_steps, "model": getattr(model, "name", type(model).__name__),
                           "n_atoms": int(positions.shape[0])}
        self.integrator = GPUNoseHooverChainNVT(
            masses, positions, np.asarray(momenta, dtype=np.float64), temperature_K=temperature,
            timestep=timestep * units.fs, tdamp=tdamp * units.fs, tchain=tchain, tloop=tloop, device=self.device,
            force_dtype=torch.float32)
        topology = model.topology_spec()
        self.cutoff = float(topology.cutoff)
        # a three-body model reads the line graph of bonds shorter than this (None: edges only)
        self.triplet_cutoff = None if topology.triplet_cutoff is None else float(topology.triplet_cutoff)
        self.graph_builder = TensorGraphBuilder(cell=self.cell, atomic_numbers=self.numbers,
                                                atom_graph_cutoff=self.cutoff, line_graph_cutoff=None,
                                                device=self.device, check_isolated_atoms=False)
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
        # F(q0) for the first pre-force half (a restart's cached evaluation: no re-evaluation)
        if restart is not None:
            self._load_restart(restart)
        else:
            forces, energy = self.evaluate(self.integrator.positions)
            self.integrator.set_forces(forces, energy=energy)
        # outputs: the trajectory / text logger and the thermo, frame and restart files
        from fastmd_amd.execution.gpu_logging import AsyncGPUMDLogger, AtomsTemplate
        from fastmd_amd.execution.md_protocol import MDOutputs

        self.logger = AsyncGPUMDLogger(
            AtomsTemplate(np.asarray(numbers), np.asarray(masses, np.float64), np.asarray(cell, np.float64),
                          np.ones(3, bool), self.explicit_masses), self.device, trajectory=trajectory, logfile=logfile,
            loginterval=loginterval, append_trajectory=append_trajectory, ring=logger_ring,
            state_dtype=torch.float64, extras={"nhc_eta": int(tchain), "nhc_p_eta": int(tchain)})
        self.outputs = MDOutputs(self, output_dir, thermo_interval, xyz_interval, restart_interval, total_steps,
                                 None if restart is None else restart.offsets, engine="native")
        if self.logger.should_log(self.steps) and restart is None:
            self._log_current()
        if self.execution == "whole_step":
            try:
                self.enable_whole_step_cuda_graph()
            except Exception as error:  # noqa: BLE001 (an out-of-memory error in auto mode only)
                if not (self.auto and _is_out_of_memory(error)):
                    raise
                self._whole_step_to_eager(error)

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
        self._after_steps()

    # ------------------------------------------------------------------ outputs
    @property
    def nsteps(self) -> int:
        return self.steps

    def _output_due(self, step: int) -> bool:
        return self.logger.should_log(step) or self.outputs.due(step)

    def _log_current(self) -> None:
        th = self.integrator
        self.logger.enqueue(step=self.steps, time_ps=self.steps * self.timestep_fs / 1000.0, positions=th.positions,
                            momenta=th.momenta, forces=th.forces, cell=self.cell, potential_energy=th.potential_energy,
                            kinetic_energy=th.kinetic_energy(), temperature=th.temperature(),
                            extras={"nhc_eta": th.eta, "nhc_p_eta": th.p_eta})

    def _after_steps(self) -> None:
        """The logger's frame and the output files due at the current step."""
        if self.logger.should_log(self.steps):
            self._log_current()
        self.outputs.write()

    def write_outputs(self) -> dict | None:
        return self.outputs.write()

    def log_frame(self, thermo: dict | None = None) -> None:
        self.outputs.log_frame(thermo)

    def save_restart(self, path=None) -> None:
        self.outputs.save_restart(path)

    def md_fields(self) -> dict:
        """Views of the current state for output and restart (gpu_md.py:2118-2140), ids = arange(N)."""
        th = self.integrator
        if getattr(self, "_masses64", None) is None:
            self._masses64 = torch.as_tensor(np.asarray(self.masses, np.float64), device=self.device)
            table = self.adapter.reference_energies() if hasattr(self.adapter, "reference_energies") else None
            ref = 0.0 if table is None else float(torch.nan_to_num(table[0, self.numbers.long() - 1]).sum())
            self._reference_energy = torch.tensor(ref, dtype=torch.float32, device=self.device)
        return {"ids": torch.arange(self.n_atoms, device=self.device), "numbers": self.numbers.to(self.device),
                "positions": th.positions, "momenta": th.momenta, "masses": self._masses64, "forces": th.forces,
                "energy": th.potential_energy.reshape(()), "reference_energy": self._reference_energy}

    def thermostat_state(self) -> dict:
        return self.integrator.state_dict()

    def collective_check(self, error: str | None) -> None:
        if error:
            raise ValueError(f"GPUResidentMolecularDynamics outputs: {error}")

    def close(self) -> None:
        """Flush and close the logger and the output files."""
        try:
            self.logger.close()
        finally:
            self.outputs.close()

    def _load_restart(self, restart) -> None:
        if restart.numbers.shape[0] != self.n_atoms or not np.array_equal(restart.numbers, self.numbers.numpy()):
            raise ValueError("the restart file's atoms are not this system's")
        th = self.integrator
        if restart.nhc_state is not None:
            th.load_state_dict(restart.nhc_state)
        th.set_state(positions=restart.positions, momenta=restart.momenta, forces=restart.forces,
                     potential_energy=np.asarray(restart.energy, np.float64).reshape(1))
        self.steps = int(restart.step)

    @classmethod
    def from_restart(cls, restart, model, **kwargs) -> "GPUResidentMolecularDynamics":
        """Continue a run from a restart file (or RestartData): its atoms, state, thermostat and
        step, the output files truncated to its offsets; the MD parameters come from ``kwargs``
        (``resume_mismatch`` lists what changed)."""
        from fastmd_amd.execution.md_protocol import read_restart
        from fastmd_amd.systems import System

        data = read_restart(restart) if not hasattr(restart, "positions") else restart
        system = System(positions=np.asarray(data.positions, np.float64), cell=np.asarray(data.cell, np.float64),
                        numbers=np.asarray(data.numbers), masses=np.asarray(data.masses, np.float64))
        return cls(system, model=model, momenta=np.asarray(data.momenta, np.float64), restart=data, **kwargs)

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
                                         padding=self.adapter.padding_rule(), n_dummy=self.config.capacity.n_dummy,
                                         prepare=prepare, device=self.device)

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

    def _whole_step_to_eager(self, error: BaseException) -> None:
        """execution="auto": an out-of-memory error while capturing a whole-step window continues
        on the eager path from the integrator's state, which the capture restored and a capacity
        overflow rolled back to its window's start (gpu_md.py:1755-1774). The runner, its graph and
        its pool are released."""
        import gc
        import warnings

        runner = self.whole_step_runner
        if runner is not None:
            for key, value in runner.stats().items():
                if key in _CUMULATIVE_STATS:
                    self._retired_stats[key] = self._retired_stats.get(key, 0) + value
        self.whole_step_runner = None
        self._graph_pool = None
        self.execution = "eager"
        del runner
        gc.collect()
        torch.cuda.empty_cache()
        self.auto_reason = f"whole_step ran out of GPU memory ({str(error).splitlines()[0][:160]}); eager"
        warnings.warn(self.auto_reason, RuntimeWarning, stacklevel=3)

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

    @roctx_ranged("md_run")
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
                if (self.launch_behind and done + 1 < windows and runner.refresh_unlikely()
                        and not self._output_due(self.steps + self.steps_per_launch)):
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
                    try:
                        self._grow_whole_step_runner(overflow.edge_count, overflow.triplet_count)
                    except Exception as error:  # noqa: BLE001 (an out-of-memory error in auto mode only)
                        if not (self.auto and _is_out_of_memory(error)):
                            raise
                        # the overflowed window was rolled back to its start: the rest eagerly
                        self._whole_step_to_eager(error)
                        for _ in range((windows - done) * self.steps_per_launch):
                            self.step()
                        return
                    continue
                done += 1
                self.steps += self.steps_per_launch
                self._after_steps()
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
        """Observables of the current state, one download (gpu_md.py:2169-2204): step, time_fs,
        target_temperature, potential / kinetic / total energy, temperature, momentum (the total),
        dof, eta, p_eta, thermostat_energy and conserved_energy (ASE's get_conserved_energy)."""
        th = self.integrator
        values = torch.cat([th.potential_energy.reshape(1).to(torch.float64), th.kinetic_energy().reshape(1),
                            th.temperature().reshape(1).to(torch.float64),
                            th.momenta.to(torch.float64).sum(0), th.eta.reshape(-1), th.p_eta.reshape(-1),
                            th.thermostat_energy().reshape(1).to(torch.float64)]).tolist()
        tchain = self.parameters["tchain"]
        potential, kinetic, temperature = values[0], values[1], values[2]
        energy = values[6 + 2 * tchain]
        return {"step": self.steps, "time_fs": self.steps * self.timestep_fs,
                "target_temperature": float(th.temperature_K), "potential_energy": potential,
                "kinetic_energy": kinetic, "total_energy": potential + kinetic, "temperature": temperature,
                "momentum": values[3:6], "dof": 3 * self.n_atoms, "eta": values[6:6 + tchain],
                "p_eta": values[6 + tchain:6 + 2 * tchain], "thermostat_energy": energy,
                "conserved_energy": potential + kinetic + energy}

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
