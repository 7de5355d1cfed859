"""Different systems in slots of one whole-step graph (fastmd/execution/system_batch.py:1-1051,
fastmd/interfaces/multi_system_md.py).

The heterogeneous counterpart of replica batching. S systems, each with its own atoms, cell,
positions, momenta and thermostat, run as one disjoint union of **slots**.
* Slot s owns the union rows [start_s, start_s + ceiling_s). Its system occupies the first
  n_s <= ceiling_s of them. The other rows are vacant: parked at the origin, no candidate, no real
  edge, no energy counted, never moved.
* A system of at most the slot's ceiling can be swapped into the slot (``write_system``): its
  positions, species, cell and a fresh chain, in the same union rows. The window graph is then
  recaptured, because its chain launches hold each system's atom count; the reference's size-class
  launches avoid that recapture.

The single-system whole-step runner runs the union unchanged; these parts make it batch-aware:
* ``SlotUnionGraphBuilder``: the fixed-capacity builder over the slots. Each system's wrap and
  candidate search run on its own slot with its own cell (the search stores union indices), so no
  edge joins two systems. The per-step build is one launch sequence over the union in which every
  row wraps with its system's cell and the padded rows take their system's far self-loop image
  (``fmd_nl_build`` with ``system_of``). It publishes the systems on ``batch.systems``
  (``SystemSegments``); the models form each edge's image in its centre's cell.
* ``SystemNoseHooverChainNVT``: one ASE-exact chain per system (the single-system kernels on the
  system's occupied rows, with its own atom count's constants), one union state for the window
  transactions. Its ``energy_segments`` make the engine derivative sum one float64 energy per system
  over its occupied rows.
* ``SystemBatchedMD``: the driver (capacity growth, replays, per-system observables).

A system's trajectory is bitwise its single-system run whenever every launch over the union takes
the form the single run takes (tested for Morse, the MACE-like and the three-body model on unions of
a few hundred rows). Launches whose form follows the system size follow each system's own atom
count (the message kernels' waves per atom, per slot); the node GEMMs take their form from the
launch's row count (fp32 tiles below a size threshold, the split-plane form above it, about 4 000
rows for the MACE-like model), so in a union that crosses the threshold a small system's node
products round differently and its trajectory matches its single run to float32 rounding instead
(tested: a 135-atom system beside the 5 000-atom perovskite, which itself stays bitwise).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from fastmd_amd import _abi, units
from fastmd_amd.adapters.protocol import SystemSegments
from fastmd_amd.config import InferenceConfig
from fastmd_amd.engine.capacity_policy import JointCapacityPolicy, held_demand, whole_step_headroom
from fastmd_amd.execution.cuda_graph import triplet_demand
from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT, NHCState, maxwell_boltzmann_momenta
from fastmd_amd.execution.whole_step_cuda_graph import FixedCapacityOverflow, WholeStepGraphRunner
from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder, morton_order, self_loop_padding
from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder
from fastmd_amd.graph.neighbor_list_backend import cell_list_shape


@dataclass(frozen=True)
class SlotLayout:
    """Slot s is the union rows [starts[s], starts[s] + ceilings[s]); fixed for the life of the
    union's captured graphs (system_batch.py:117-147)."""

    ceilings: tuple

    def __post_init__(self) -> None:
        if not self.ceilings or any(int(c) <= 0 for c in self.ceilings):
            raise ValueError("every slot needs a positive ceiling")

    @property
    def count(self) -> int:
        return len(self.ceilings)

    @property
    def starts(self) -> tuple:
        return tuple(int(x) for x in np.concatenate([[0], np.cumsum(self.ceilings)[:-1]]))

    @property
    def rows(self) -> int:
        return int(sum(self.ceilings))


def _cell32(cell) -> np.ndarray:
    cell = np.asarray(cell, dtype=np.float64)
    if cell.shape != (3, 3) or not np.isfinite(cell).all() or abs(np.linalg.det(cell)) < 1e-6:
        raise ValueError("a system cell must be a finite, non-singular 3 x 3 matrix (rows = lattice vectors)")
    return cell.astype(np.float32)


class SlotUnionGraphBuilder(FixedCapacityGraphBuilder):
    """The edges-only (or line-graph) fixed-capacity builder over the slots of a union
    (system_batch.py:177-444). ``cells``: one 3 x 3 cell per slot; ``atomic_numbers``: the union
    rows (a vacant row any supported number); ``atoms``: each slot's occupied rows."""

    def __init__(self, *, layout: SlotLayout, cells, atomic_numbers, atoms, u_capacity: int, t_capacity: int = 0,
                 atom_graph_cutoff: float = 6.0, line_graph_cutoff: float | None = None,
                 candidate_cutoff: float | None = None, padding=None, prepare=None,
                 device: torch.device | str = "cuda", minimum_image: bool = False) -> None:
        if padding is not None and padding.kind == "sink_atoms":
            raise NotImplementedError("a slot union pads with self-loops (sink rows would sit between slots)")
        cells32 = [_cell32(c) for c in cells]
        atoms = [int(a) for a in atoms]
        if len(cells32) != layout.count or len(atoms) != layout.count:
            raise ValueError("one cell and one atom count per slot")
        if any(not 0 < a <= c for a, c in zip(atoms, layout.ceilings)):
            raise ValueError("each slot holds between 1 and its ceiling of atoms")
        numbers = torch.as_tensor(atomic_numbers, dtype=torch.int32).reshape(-1)
        if numbers.numel() != layout.rows:
            raise ValueError(f"atomic_numbers must cover the {layout.rows} union rows")
        super().__init__(cell=torch.from_numpy(cells32[0]), atomic_numbers=numbers, u_capacity=u_capacity,
                         t_capacity=t_capacity, atom_graph_cutoff=atom_graph_cutoff,
                         line_graph_cutoff=line_graph_cutoff, candidate_cutoff=candidate_cutoff, padding=padding,
                         device=device, minimum_image=minimum_image)
        self.layout = layout
        dev = self.device
        self.atoms = atoms
        self._sys_cells = torch.empty((layout.count, 3, 3), dtype=torch.float32, device=dev)
        self._sys_inv = torch.empty_like(self._sys_cells)
        self._pad_images = torch.empty((layout.count, 3), dtype=torch.int32, device=dev)
        self._shapes = [None] * layout.count
        self._cell_lists = [None] * layout.count
        self._sys_valid = torch.ones(layout.count, dtype=torch.uint8, device=dev)
        system_of = np.repeat(np.arange(layout.count, dtype=np.int32), layout.ceilings)
        self._system_of = torch.tensor(system_of, dtype=torch.int32, device=dev)
        self._row_ptr = torch.tensor(np.concatenate([layout.starts, [layout.rows]]), dtype=torch.int64, device=dev)
        self._atoms = torch.tensor(atoms, dtype=torch.int64, device=dev)
        for s, c in enumerate(cells32):
            self._set_cell(s, c)
        # the published cell is the per-system table; the builder's one-cell state is not used
        self.cell, self.inv_cell = self._sys_cells, self._sys_inv
        self.batch.cell = self._sys_cells
        self.batch.systems = SystemSegments(count=layout.count, row_ptr=self._row_ptr,
                                            system_of_row=self._system_of, cells=self._sys_cells, atoms=self._atoms)
        self.batch.max_system_rows = max(layout.ceilings)
        self.batch.system_slots = tuple(zip(layout.starts, layout.ceilings, atoms))
        self.graph = self.batch if prepare is None else prepare(self.batch)

    def _set_cell(self, slot: int, cell32: np.ndarray) -> None:
        """Slot ``slot``'s cell, its inverse (of the float32 cell, in float64, rounded to float32: the
        single-system builder's), its far self-loop image and its cell-list shape and buffers."""
        if cell32.shape != (3, 3):
            raise ValueError("a cell is 3 x 3")
        ceiling = self.layout.ceilings[slot]
        heights = 1.0 / np.linalg.norm(np.linalg.inv(cell32.astype(np.float64)), axis=0)
        if np.any(heights < 1e-3):
            raise ValueError("degenerate cell")
        self._sys_cells[slot].copy_(torch.from_numpy(cell32))
        self._sys_inv[slot].copy_(torch.from_numpy(np.linalg.inv(cell32.astype(np.float64)).astype(np.float32)))
        image = self_loop_padding(self.padding, torch.from_numpy(cell32), self.atom_graph_cutoff)[0]
        self._pad_images[slot].copy_(torch.tensor(image, dtype=torch.int32))
        shape = cell_list_shape(cell32, self.candidate_cutoff)
        ncell = shape[0][0] * shape[0][1] * shape[0][2]
        i32 = dict(dtype=torch.int32, device=self.device)
        self._shapes[slot] = shape
        self._cell_lists[slot] = (torch.zeros(ncell, **i32), torch.zeros(ncell + 1, **i32), torch.zeros(ceiling, **i32))

    def _slice_ptr(self, t: Tensor, start: int, per_row: int) -> int:
        return t.data_ptr() + start * per_row * t.element_size()

    @torch.no_grad()
    def refresh_candidates(self, positions: Tensor) -> None:
        """Each slot's wrap (all its rows: vacant rows get a reference too) and candidate search over
        its occupied rows in its own cell, storing union indices; the union's capacity flag is every
        slot's."""
        positions = self._positions_arg(positions)
        is64 = 1 if positions.dtype == torch.float64 else 0
        stream = self._stream()
        bmax = self.buffer_max
        for s, (start, ceiling) in enumerate(zip(self.layout.starts, self.layout.ceilings)):
            cell = self._sys_cells[s].data_ptr()
            inv = self._sys_inv[s].data_ptr()
            _abi.call("fmd_nl_wrap", self._slice_ptr(positions, start, 3), is64, inv, cell, ceiling,
                      self._slice_ptr(self.frac_coords, start, 3), self._slice_ptr(self._wraps, start, 3),
                      self._slice_ptr(self._wrapped_refresh, start, 3),
                      self._slice_ptr(self.reference_positions, start, 3),
                      self._slice_ptr(self.reference_wraps, start, 3), self._slice_ptr(self.wrap_delta, start, 3),
                      stream)
            (ncells, reach), (count, first, members) = self._shapes[s], self._cell_lists[s]
            _abi.call("fmd_nl_candidates", self._slice_ptr(self._wrapped_refresh, start, 3),
                      self._slice_ptr(self.frac_coords, start, 3), cell, self.atoms[s], self._cand2,
                      _abi.array(_abi._i32, ncells), _abi.array(_abi._i32, reach), bmax, count.data_ptr(),
                      first.data_ptr(), members.data_ptr(), self._slice_ptr(self.neighbor_matrix, start, bmax),
                      self._slice_ptr(self.neighbor_shifts, start, 3 * bmax),
                      self._slice_ptr(self.num_neighbors, start, 1), self._sys_valid[s:s + 1].data_ptr(), 0, start,
                      stream)
        torch.amin(self._sys_valid, dim=0, keepdim=True, out=self._candidate_capacity_valid)
        self.atom_order.copy_(morton_order(self.frac_coords, self._system_of))
        self._candidate_owner._candidate_initialized = True


@dataclass
class SystemNHCState:
    """Views into one flat float64 buffer: the union rows and per-system chains and energies."""

    flat: Tensor
    positions: Tensor  # [rows, 3]
    momenta: Tensor
    forces: Tensor
    eta: Tensor  # [systems, tchain]
    p_eta: Tensor
    potential_energy: Tensor  # [systems]

    @staticmethod
    def allocate(rows: int, systems: int, tchain: int, device) -> "SystemNHCState":
        flat = torch.zeros(9 * rows + 2 * systems * tchain + systems, dtype=torch.float64, device=device)
        o, views = 0, []
        for size, shape in ((3 * rows, (rows, 3)), (3 * rows, (rows, 3)), (3 * rows, (rows, 3)),
                            (systems * tchain, (systems, tchain)), (systems * tchain, (systems, tchain)),
                            (systems, (systems,))):
            views.append(flat[o:o + size].view(*shape))
            o += size
        return SystemNHCState(flat, *views)

    def system(self, s: int, start: int, atoms: int) -> NHCState:
        rows = slice(start, start + atoms)
        return NHCState(None, self.positions[rows], self.momenta[rows], self.forces[rows], self.eta[s],
                        self.p_eta[s], self.potential_energy[s:s + 1])


class SystemNoseHooverChainNVT:
    """One ASE-exact Nose-Hoover chain per system (a ``GPUNoseHooverChainNVT`` on the system's
    occupied rows, with its own atom count's constants) over one union state; the whole-step
    runner's integrator protocol on the union rows (system_batch.py:563-792)."""

    ensemble = "nvt_nhc"

    def __init__(self, layout: SlotLayout, masses, positions, momenta, *, temperature_K: float, timestep: float,
                 tdamp: float, tchain: int = 3, tloop: int = 1, device="cuda",
                 force_dtype: torch.dtype = torch.float32) -> None:
        self.layout = layout
        self.systems = layout.count
        self.n_atoms = layout.rows
        self.tchain = int(tchain)
        self.device = torch.device(device)
        self._params = dict(temperature_K=temperature_K, timestep=timestep, tdamp=tdamp, tchain=tchain, tloop=tloop,
                            device=device, force_dtype=force_dtype)
        self.state = SystemNHCState.allocate(self.n_atoms, self.systems, self.tchain, self.device)
        self._backup = SystemNHCState.allocate(self.n_atoms, self.systems, self.tchain, self.device)
        self.masses = torch.ones(self.n_atoms, 1, dtype=torch.float64, device=self.device)  # vacant rows: 1
        self._subs = [None] * self.systems
        self.atoms = [0] * self.systems
        for s in range(self.systems):
            self.write_system(s, masses=masses[s], positions=positions[s], momenta=momenta[s])

    def write_system(self, slot: int, *, masses, positions, momenta) -> None:
        """The system in ``slot``: its chain starts fresh (ASE's initial state) from ``positions`` and
        ``momenta``; the slot's vacant rows are parked at the origin at rest."""
        masses = np.asarray(masses, np.float64).reshape(-1)
        n = int(masses.shape[0])
        start, ceiling = self.layout.starts[slot], self.layout.ceilings[slot]
        if not 0 < n <= ceiling:
            raise ValueError(f"slot {slot} holds at most {ceiling} atoms")
        sub = GPUNoseHooverChainNVT(masses, np.asarray(positions, np.float64).reshape(n, 3),
                                    np.asarray(momenta, np.float64).reshape(n, 3), **self._params)
        rows = slice(start, start + ceiling)
        for name in ("positions", "momenta", "forces"):
            getattr(self.state, name)[rows].zero_()
        self.masses[rows] = 1.0
        self.masses[start:start + n] = sub.masses.reshape(n, 1)
        view = self.state.system(slot, start, n)
        for name in ("positions", "momenta", "forces", "eta", "p_eta", "potential_energy"):
            getattr(view, name).copy_(getattr(sub.state, name))
        sub.state = view  # the chain integrates its system's rows of the union state
        self._subs[slot] = sub
        self.atoms[slot] = n

    @property
    def energy_segments(self) -> tuple:
        """(start, atoms) of every system: the engine derivative's per-system energy ranges."""
        return tuple((start, n) for start, n in zip(self.layout.starts, self.atoms))

    @property
    def temperature_K(self) -> float:
        return self._subs[0].temperature_K

    def set_temperature(self, temperature_K: float) -> None:
        for sub in self._subs:
            sub.set_temperature(temperature_K)
        self._params["temperature_K"] = temperature_K

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

    def system(self, s: int) -> GPUNoseHooverChainNVT:
        return self._subs[s]

    @torch.no_grad()
    def set_state(self, *, positions=None, momenta=None, forces=None, potential_energy=None) -> None:
        st = self.state
        for name, value in (("positions", positions), ("momenta", momenta), ("forces", forces)):
            if value is not None:
                getattr(st, name).copy_(torch.as_tensor(value, dtype=torch.float64, device=self.device)
                                        .reshape(self.n_atoms, 3))
        if potential_energy is not None:
            st.potential_energy.copy_(torch.as_tensor(potential_energy, dtype=torch.float64,
                                                      device=self.device).reshape(self.systems))

    def set_forces(self, forces, energy=None) -> None:
        for sub, (start, n) in zip(self._subs, self.energy_segments):
            sub.state.forces.copy_(forces.reshape(self.n_atoms, 3)[start:start + n])
        if energy is not None:
            self.state.potential_energy.copy_(energy.reshape(self.systems).to(torch.float64))

    def step_pre_force(self) -> Tensor:
        for sub in self._subs:
            sub.step_pre_force()
        return self.state.positions

    def step_post_force(self, forces: Tensor, energy: Tensor | None = None) -> None:
        forces = forces.reshape(self.n_atoms, 3)
        energy = None if energy is None else energy.reshape(-1)
        if energy is not None and energy.numel() != self.systems:
            raise ValueError(f"one energy per system expected, got {energy.numel()}")
        for s, (sub, (start, n)) in enumerate(zip(self._subs, self.energy_segments)):
            sub.step_post_force(forces[start:start + n], energy=None if energy is None else energy[s:s + 1])

    # transactions on the union state
    def backup(self, state: SystemNHCState | None = None) -> None:
        self._backup.flat.copy_((self.state if state is None else state).flat)

    def restore(self, state: SystemNHCState | None = None) -> None:
        (self.state if state is None else state).flat.copy_(self._backup.flat)

    def snapshot(self) -> tuple:
        return self.state.flat.clone(), self._backup.flat.clone()

    def load_snapshot(self, snapshot: tuple) -> None:
        state, backup = snapshot
        self.state.flat.copy_(state)
        self._backup.flat.copy_(backup)

    def new_state(self) -> SystemNHCState:
        return SystemNHCState.allocate(self.n_atoms, self.systems, self.tchain, self.device)

    # observables per system
    def kinetic_energy(self) -> Tensor:
        return torch.stack([sub.kinetic_energy() for sub in self._subs])

    def temperature(self) -> Tensor:
        return torch.stack([sub.temperature() for sub in self._subs])

    def conserved_energy(self) -> Tensor:
        return torch.stack([sub.conserved_energy() for sub in self._subs])


def _system_arrays(atoms):
    from fastmd_amd.interfaces.gpu_md import _atoms_arrays

    positions, cell, numbers, masses, _ = _atoms_arrays(atoms)
    return positions, cell, np.asarray(numbers), masses


class SystemBatchedMD:
    """S different systems (own atoms, cells, momenta and thermostats) in slots of one whole-step
    graph per window: ``GPUResidentMolecularDynamics``'s parameters plus ``ceilings`` (rows per slot,
    default each system's atom count) and per-system ``seeds`` or ``momenta``; ``run(steps)``,
    per-system ``thermodynamics()`` and ``system_state(s)``, ``write_system`` to swap a system into
    a slot."""

    def __init__(self, systems, model, *, ceilings=None, device: torch.device | str = "cuda",
                 temperature: float = 300.0, timestep: float = 1.0, tdamp: float = 100.0, tchain: int = 3,
                 tloop: int = 1, seeds=None, momenta=None, steps_per_launch: int = 1,
                 config: InferenceConfig | None = None) -> None:
        self.config = config or InferenceConfig()
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.adapter = model
        self.steps_per_launch = int(steps_per_launch)
        arrays = [_system_arrays(a) for a in systems]
        counts = [int(p.shape[0]) for p, _, _, _ in arrays]
        self.layout = SlotLayout(tuple(counts if ceilings is None else (int(c) for c in ceilings)))
        if self.layout.count != len(arrays):
            raise ValueError("one ceiling per system")
        if momenta is None:
            seeds = list(range(len(arrays))) if seeds is None else list(seeds)
            momenta = [maxwell_boltzmann_momenta(m, temperature, sd) for (_, _, _, m), sd in zip(arrays, seeds)]
        self.timestep_fs = float(timestep)
        self.integrator = SystemNoseHooverChainNVT(
            self.layout, [m for _, _, _, m in arrays], [p for p, _, _, _ in arrays], momenta,
            temperature_K=temperature, timestep=timestep * units.fs, tdamp=tdamp * units.fs, tchain=tchain,
            tloop=tloop, device=self.device)
        numbers = np.zeros(self.layout.rows, dtype=np.int32)
        for start, ceiling, (_, _, z, _) in zip(self.layout.starts, self.layout.ceilings, arrays):
            numbers[start:start + ceiling] = z[0]
            numbers[start:start + len(z)] = z
        self.numbers = torch.tensor(numbers)
        self.cells = [np.asarray(c, np.float64) for _, c, _, _ in arrays]
        self.atoms = counts
        topology = model.topology_spec()
        self.cutoff = float(topology.cutoff)
        self.triplet_cutoff = None if topology.triplet_cutoff is None else float(topology.triplet_cutoff)
        u, t = self._demand(arrays)
        step = model.capacity_step() if hasattr(model, "capacity_step") else None
        cap = self.config.capacity
        self._u_step, self._min_pad = (step.u_step, step.min_pad_u) if step is not None else (cap.u_step, cap.min_pad_u)
        self._factors = (step.u_thermal_factor, step.t_thermal_factor) if step is not None else (1.0, 1.0)
        self._t_step = (step.t_step or 128) if step is not None else cap.t_step
        self.policy = JointCapacityPolicy(u_step=self._u_step, min_pad_u=self._min_pad,
                                          t_step=self._t_step if self.triplet_cutoff is not None else None,
                                          min_pad_t=(step.min_pad_t if step is not None else cap.min_pad_t))
        self._capacity = self.policy.start(*self._held(u, t))
        self._pool = torch.cuda.graph_pool_handle()
        self.steps = 0
        self.runner = None
        self.capacity_history = []
        self._make_runner(recapture=False)

    def _demand(self, arrays) -> tuple[int, int]:
        """The union's pair and triplet demand: the sum of each system's ragged build."""
        u = t = 0
        for positions, cell, numbers, _ in arrays:
            single = TensorGraphBuilder(cell=torch.tensor(cell, dtype=torch.float64),
                                        atomic_numbers=torch.tensor(numbers, dtype=torch.int32),
                                        atom_graph_cutoff=self.cutoff, line_graph_cutoff=None, device=self.device,
                                        check_isolated_atoms=False)
            sample = single.build(torch.as_tensor(positions, dtype=torch.float64, device=self.device))
            u += int(sample.edge_index.shape[0]) // 2
            if self.triplet_cutoff is not None:
                t += triplet_demand(sample, self.triplet_cutoff)
        return u, t

    def _held(self, u: int, t: int) -> tuple[int, int]:
        uf, tf = self._factors
        hu = held_demand(u, whole_step_headroom(u, self._u_step), uf)
        ht = held_demand(t, whole_step_headroom(t, self._t_step), tf) if self.triplet_cutoff is not None else 0
        return hu, ht

    def _builder(self, key) -> SlotUnionGraphBuilder:
        return SlotUnionGraphBuilder(
            layout=self.layout, cells=self.cells, atomic_numbers=self.numbers, atoms=self.atoms,
            u_capacity=key.u_capacity, t_capacity=key.t_capacity if self.triplet_cutoff is not None else 0,
            atom_graph_cutoff=self.cutoff, line_graph_cutoff=self.triplet_cutoff,
            candidate_cutoff=self.cutoff + self.config.capacity.candidate_skin, padding=self.adapter.padding_rule(),
            prepare=self.adapter.prepare, device=self.device)

    def _make_runner(self, recapture: bool) -> None:
        while True:
            key = self._capacity
            try:
                self.runner = WholeStepGraphRunner(model=self.adapter, builder=self._builder(key),
                                                   integrator=self.integrator, steps_per_launch=self.steps_per_launch,
                                                   warmup=self.config.capacity.warmup, graph_pool=self._pool,
                                                   recapture=recapture)
                self.capacity_history.append((key.u_capacity, key.t_capacity))
                return
            except FixedCapacityOverflow as overflow:
                self._grow(overflow)

    def _grow(self, overflow: FixedCapacityOverflow) -> None:
        self._capacity = self.policy.grow(self._capacity, *self._held((overflow.edge_count + 1) // 2,
                                                                      overflow.triplet_count))

    def run(self, steps: int) -> None:
        """``steps`` MD steps of every system (a multiple of ``steps_per_launch``)."""
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

    def write_system(self, slot: int, atoms, *, momenta=None, seed: int = 0) -> None:
        """Swap another system (at most the slot's ceiling of atoms, any cell) into ``slot`` between
        windows: species, cell, positions, momenta (Maxwell-Boltzmann at the target temperature from
        ``seed`` by default) and a fresh chain. The union's rows stay those of the layout; the window
        graph is recaptured (its chain launches hold each system's atom count), at the current
        capacity or a grown one."""
        positions, cell, numbers, masses = _system_arrays(atoms)
        n = int(positions.shape[0])
        if not 0 < n <= self.layout.ceilings[slot]:
            raise ValueError(f"slot {slot} holds at most {self.layout.ceilings[slot]} atoms")
        _cell32(cell)
        if momenta is None:
            momenta = maxwell_boltzmann_momenta(masses, self.integrator.temperature_K, seed)
        self.integrator.write_system(slot, masses=masses, positions=positions, momenta=momenta)
        self.cells[slot] = np.asarray(cell, np.float64)
        self.atoms[slot] = n
        start, ceiling = self.layout.starts[slot], self.layout.ceilings[slot]
        self.numbers[start:start + ceiling] = int(numbers[0])
        self.numbers[start:start + n] = torch.as_tensor(numbers, dtype=torch.int32)
        self.runner = None
        self._make_runner(recapture=True)

    def system_state(self, s: int) -> dict:
        """Views of system s's positions, momenta and forces (float64 [n_s, 3]) and its energy."""
        start, n = self.integrator.energy_segments[s]
        st = self.integrator.state
        rows = slice(start, start + n)
        return {"positions": st.positions[rows], "momenta": st.momenta[rows], "forces": st.forces[rows],
                "potential_energy": st.potential_energy[s]}

    def thermodynamics(self) -> list[dict]:
        """Per system: step, potential / kinetic / total energy, temperature, conserved energy."""
        th = self.integrator
        epot = th.potential_energy.tolist()
        ekin = th.kinetic_energy().tolist()
        temp = th.temperature().tolist()
        cons = th.conserved_energy().tolist()
        return [{"step": self.steps, "time_fs": self.steps * self.timestep_fs, "atoms": self.atoms[s],
                 "potential_energy": epot[s], "kinetic_energy": ekin[s], "total_energy": epot[s] + ekin[s],
                 "temperature": temp[s], "conserved_energy": cons[s]} for s in range(self.layout.count)]

    def stats(self) -> dict:
        st = self.runner.stats()
        st["capacity_history"] = list(self.capacity_history)
        st["layout"] = list(self.layout.ceilings)
        return st
