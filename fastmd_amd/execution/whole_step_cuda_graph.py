"""(f) The whole MD step captured as ONE hipGraph and replayed per window.

Same contract as the reference's ``WholeStepGraphRunner``
(fastmd/execution/whole_step_cuda_graph.py:56-736) for a stateful (NHC) integrator and an
edges-only builder: a window is a transaction -- the integrator's one-copy backup, the window
flags reset, then ``steps_per_launch`` x (``step_pre_force`` -> exact re-filter build ->
engine-owned derivative -> ``step_post_force`` -> flag fold) -- captured once (after
side-stream warmup windows that are rolled back) and replayed; after a replay the host reads
one small statistics buffer and settles the window:

* capacity overflow (edges > e_cap): roll back and raise ``FixedCapacityOverflow`` (the driver
  grows the capacity and recaptures);
* an invalid candidate list (an atom moved more than half the skin, or a truncated row): roll
  back, refresh the candidates at the window's start state and replay (recovery), falling back
  to eager steps with fresh candidates if that fails again;
* a proactive candidate refresh when the largest displacement reached
  ``proactive_refresh_fraction`` of the skin;
* non-finite state (NaN displacement) raises.

Every kernel of the body is a HIP kernel of this package launched on torch's current stream
(captured by torch.cuda.CUDAGraph = hipStreamBeginCapture/hipGraphInstantiate); the flags are
cleared by fill kernels, never memsets.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import Tensor

from fastmd_amd.engine.energy_derivative import engine_derivative
from fastmd_amd.execution.graph_capture import capture_graph
from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder
from fastmd_amd.graph.gpu_graph_builder import raise_if_isolated_atoms
from fastmd_amd._roctx import roctx_ranged


def _capacity_exceeded(builder, status) -> bool:
    """A build's capacity overflow, read on the host (initial evaluation): edges above e_capacity;
    for a line-graph build also edges at e_capacity, invalid pairs or triplets above t_capacity."""
    edges = int(status.edge_count.item())
    if builder.line_graph is None:
        return edges > builder.e_capacity
    return (edges >= builder.e_capacity or bool(status.invalid_pairs.item())
            or int(status.triplet_count.item()) > builder.t_capacity)


class FixedCapacityOverflow(RuntimeError):
    def __init__(self, edge_count: int, triplet_count: int = 0) -> None:
        super().__init__(f"fixed graph capacity exceeded: edges={edge_count}, triplets={triplet_count}")
        self.edge_count = edge_count
        self.triplet_count = triplet_count


def _require_finite_displacement(displacement: float, launch: int) -> None:
    """whole_step_cuda_graph.py:25-35: NaN positions show as a NaN maximum displacement."""
    if not math.isfinite(displacement):
        raise ValueError(f"non-finite MD state after whole-step launch {launch}: max displacement {displacement}")


@dataclass
class WindowStats:
    overflow: bool
    edge_count: int
    max_displacement: float
    capacity_overflow: bool
    max_edges: int
    max_isolated: int
    max_triplets: int = 0


class WholeStepGraphRunner:
    """Capture integrator + exact graph re-filter + model forces (see the module docstring)."""

    def __init__(self, *, model, builder: FixedCapacityGraphBuilder, integrator, positions: Tensor | None = None,
                 momenta: Tensor | None = None, forces: Tensor | None = None, task: str = "ef",
                 steps_per_launch: int = 1, warmup: int = 3, proactive_refresh_fraction: float = 0.25,
                 graph_pool=None, validate_isolated_atoms: bool = False, config=None, recapture: bool = False,
                 capture: bool = True) -> None:
        if steps_per_launch <= 0:
            raise ValueError("steps_per_launch must be positive")
        if not 0.0 < proactive_refresh_fraction < 0.5:
            raise ValueError("proactive_refresh_fraction must be in (0, 0.5)")
        if "s" in task:
            raise NotImplementedError("stress windows are not supported")
        self.adapter = model
        self._derivative = engine_derivative(model)
        replicas = int(getattr(integrator, "replicas", 1))
        ranges = getattr(integrator, "energy_segments", None)
        if ranges is not None and self._derivative is not None:
            # a slot union of systems: one energy per system (its occupied rows)
            self._derivative.segments = tuple(ranges)
        elif replicas > 1 and self._derivative is not None:
            # a replica batch: one energy per replica for its integrator
            self._derivative.segments = replicas
        if self._derivative is None:
            raise NotImplementedError("model-owned derivatives are not supported: the model needs an EnergyTap")
        self.builder = builder
        self.integrator = integrator
        self.task = task
        self.steps_per_launch = int(steps_per_launch)
        self.warmup = 1 if recapture else int(warmup)
        self.proactive_refresh_fraction = float(proactive_refresh_fraction)
        self.graph_pool = graph_pool
        self.validate_isolated_atoms = bool(validate_isolated_atoms) or model.isolated_atom_policy() == "error"
        self.n_real = builder.n_real
        self.device = builder.device
        dev = self.device
        self.window_overflow = torch.zeros(1, dtype=torch.uint8, device=dev)
        self.window_capacity_overflow = torch.zeros(1, dtype=torch.uint8, device=dev)
        self.window_max_edges = torch.zeros(1, dtype=torch.int64, device=dev)
        self.window_max_isolated = torch.zeros(1, dtype=torch.int32, device=dev)
        self.window_max_triplets = torch.zeros(1, dtype=torch.int64, device=dev)
        self._window_stats = torch.zeros(7, dtype=torch.float64, device=dev)
        # two host slots for the statistics of launched windows (one settled while the window
        # launched behind it runs), each with the event of its copy
        self._slots = [[torch.zeros(7, dtype=torch.float64, pin_memory=True), None] for _ in range(2)]
        self._next_slot = 0
        self._last_slot = None
        # launch(behind=True): the unsettled window's start state (its integrator backup, which the
        # window behind overwrites), kept for rewind()
        self._held = None
        # what refresh_unlikely() reads: the last settled window's largest displacement, whether it
        # fell back, and the largest growth of the displacement per window with the current and the
        # previous candidate list
        self._settled_displacement = 0.0
        self._settled_fallback = False
        self._displacement_growth = [None, None]
        self.graph = None
        self.fallback_windows = 0
        self.candidate_refreshes = 0
        self.recovery_replays = 0
        self.launches = 0
        self.max_edge_count = 0
        self.max_displacement_seen = 0.0
        self.last_edge_count = 0
        self.warmup_runs = 0
        if positions is not None:
            integrator.set_state(positions=positions)
        if momenta is not None:
            integrator.set_state(momenta=momenta)
        # candidates at the current state, then the initial evaluation F(q0)
        self.builder.refresh_candidates(integrator.positions)
        self.candidate_refreshes += 1
        self.builder.assert_candidate_capacity()
        f0, e0, status = self._evaluate(integrator.positions)
        if _capacity_exceeded(builder, status):
            raise FixedCapacityOverflow(int(status.edge_count.item()), int(status.triplet_count.item()))
        if self.validate_isolated_atoms:
            raise_if_isolated_atoms(int(status.isolated_atom_count.item()))
        if forces is None:
            integrator.set_forces(f0.detach(), energy=e0.detach())
        else:
            integrator.set_forces(forces.to(device=dev, dtype=torch.float64))
        if capture:
            self._capture()

    # ------------------------------------------------------------------ body
    def _evaluate(self, positions: Tensor, window: dict | None = None):
        graph, status = self.builder.build(positions, rebuild_candidates=False, window=window)
        out = self._derivative(self.builder.batch, graph, task=self.task, n_real=self.n_real)
        forces = out["f"][0][: self.n_real]
        energy = out["e"].reshape(-1)  # one energy (or one per replica of a replica batch)
        return forces, energy, status

    def _step_body(self, last: bool, positions: Tensor | None = None, fuse_next: bool = False):
        """One step. ``positions``: this step's pre-force half already ran (fused into the step
        before). ``fuse_next``: the next step's pre-force half runs fused with this step's post-force
        half (one integrator launch); its positions are returned."""
        integrator = self.integrator
        if positions is None:
            positions = integrator.step_pre_force()
        # the window's flag fold reads only the build's status: the build does it (an edges-only
        # build in its own launch), so that the post-force half and the next pre-force half stay
        # adjacent
        window = dict(window_overflow=self.window_overflow, window_capacity_overflow=self.window_capacity_overflow,
                      window_max_edges=self.window_max_edges, window_max_isolated=self.window_max_isolated,
                      check_isolated=self.validate_isolated_atoms, stats=self._window_stats if last else None,
                      window_max_triplets=self.window_max_triplets)
        forces, energy, status = self._evaluate(positions, window)
        with torch.no_grad():
            if fuse_next:
                return integrator.step_post_pre(forces.detach(), energy=energy.detach())
            integrator.step_post_force(forces.detach(), energy=energy.detach())
        return None

    def _window_body(self) -> None:
        self.integrator.backup()
        self.window_overflow.zero_()
        self.window_capacity_overflow.zero_()
        self.window_max_edges.zero_()
        self.window_max_isolated.zero_()
        self.window_max_triplets.zero_()
        fuse = hasattr(self.integrator, "step_post_pre")
        positions = None
        for k in range(self.steps_per_launch):
            last = k == self.steps_per_launch - 1
            positions = self._step_body(last=last, positions=positions, fuse_next=fuse and not last)

    def _capture(self) -> None:
        integrator = self.integrator
        saved = integrator.snapshot()
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        try:
            with torch.cuda.stream(side):
                for _ in range(self.warmup):
                    self._window_body()
                    integrator.load_snapshot(saved)
                    self.warmup_runs += 1
            torch.cuda.current_stream(self.device).wait_stream(side)
            torch.cuda.synchronize(self.device)
            self.graph = torch.cuda.CUDAGraph()
            with capture_graph(self.graph, pool=self.graph_pool, name="whole_step_capture"):
                self._window_body()
        except BaseException:
            torch.cuda.current_stream(self.device).wait_stream(side)
            integrator.load_snapshot(saved)
            raise
        integrator.load_snapshot(saved)
        torch.cuda.synchronize(self.device)

    # ------------------------------------------------------------------ replay
    @roctx_ranged("whole_step_launch")
    def launch(self, *, behind: bool = False) -> int:
        """Replay one window without settling it and start the asynchronous copy of its statistics
        into a host slot (no host synchronization); returns the slot for :meth:`launched_stats`.
        ``behind``: the previously launched window is not settled yet; its start state, which this
        window's backup overwrites, is kept first for :meth:`rewind` (whole_step_cuda_graph.py:598-627)."""
        if behind:
            if self._held is None:
                self._held = self.integrator.new_state()
            self.integrator.restore(self._held)  # its backup (the unsettled window's start) into held
        if self.graph is None:
            self._window_body()
        else:
            self.graph.replay()
        self.launches += 1
        slot = self._next_slot
        self._next_slot ^= 1
        host = self._slots[slot][0]
        host.copy_(self._window_stats, non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        self._slots[slot][1] = event
        self._last_slot = slot
        return slot

    def launched_stats(self, slot: int) -> WindowStats:
        """The statistics of the window :meth:`launch` copied into ``slot``, once that copy is done
        (waits for that window only)."""
        host, event = self._slots[slot]
        event.synchronize()
        s = host.tolist()
        return WindowStats(bool(s[0]), int(s[1]), float(s[3]), bool(s[4]), int(s[5]), int(s[6]), int(s[2]))

    def read_stats(self) -> WindowStats:
        """Wait for the last launched window's statistics (the one host sync per window)."""
        return self.launched_stats(self._last_slot)

    def settling_work(self, stats: WindowStats) -> str | None:
        """What settling a window with these statistics changes beyond host bookkeeping
        (whole_step_cuda_graph.py:629-639): "overflow" (rollback and growth, or the fallback replay),
        "refresh" (new candidates; also a non-finite state, which raises), else None."""
        if stats.capacity_overflow or stats.overflow:
            return "overflow"
        if not math.isfinite(stats.max_displacement):
            return "refresh"
        return "refresh" if stats.max_displacement >= self.proactive_refresh_fraction * self.builder.skin else None

    def refresh_unlikely(self) -> bool:
        """Whether the window in flight will likely neither refresh the candidates nor fall back
        (whole_step_cuda_graph.py:586-596): the last settled window did not fall back, and its largest
        displacement plus twice the largest growth per window seen with this or the previous
        candidate list stays below the refresh threshold. A window launched behind one that does is
        rolled back (one window of GPU time), so the driver launches none behind a likely one."""
        growth = [g for g in self._displacement_growth if g is not None]
        if not growth or self._settled_fallback:
            return False
        threshold = self.builder.skin * self.proactive_refresh_fraction
        return self._settled_displacement + 2.0 * max(growth) < threshold

    def rewind(self) -> None:
        """Roll back the unsettled window and the one launched behind it to the unsettled window's
        start (kept by ``launch(behind=True)``), which is also the backup again: settling the
        unsettled window (its fallback or capacity rollback) then proceeds as if nothing had been
        launched behind it."""
        self.integrator.backup(self._held)  # the held start into the backup, then into the state
        self.integrator.restore()
        self.launches -= 1

    def drop(self) -> None:
        """Roll back the window launched last (behind another) to its start, the previous window's
        end."""
        self.integrator.restore()
        self.launches -= 1

    def settle(self, stats: WindowStats) -> None:
        """Act on a window's flags (whole_step_cuda_graph.py:540-584)."""
        _require_finite_displacement(stats.max_displacement, self.launches)
        self.last_edge_count = stats.edge_count
        self.max_edge_count = max(self.max_edge_count, stats.max_edges)
        self.max_displacement_seen = max(self.max_displacement_seen, stats.max_displacement)
        if stats.capacity_overflow:
            self.integrator.restore()
            raise FixedCapacityOverflow(stats.max_edges, stats.max_triplets)
        if stats.overflow:
            self._fallback()
            # fresh candidates at the window's start: the displacement restarts (an upper bound of
            # the growth follows from the next window), and none is launched behind the next one
            self._settled_fallback = True
            self._settled_displacement = 0.0
            self._displacement_growth = [None, self._displacement_growth[0]]
            return
        self._settled_fallback = False
        growth = stats.max_displacement - self._settled_displacement
        self._displacement_growth[0] = max(growth, self._displacement_growth[0] or 0.0)
        self._settled_displacement = stats.max_displacement
        if stats.max_displacement >= self.proactive_refresh_fraction * self.builder.skin:
            self.builder.refresh_candidates(self.integrator.positions)
            self.candidate_refreshes += 1
            self.builder.assert_candidate_capacity()
            self._settled_displacement = 0.0
            self._displacement_growth = [None, self._displacement_growth[0]]

    def _fallback(self) -> None:
        """Roll the window back, refresh the candidates at its start state and replay it; if the
        replay is invalid again, run its steps eagerly with a fresh candidate list per step."""
        self.fallback_windows += 1
        self.integrator.restore()
        self.builder.refresh_candidates(self.integrator.positions)
        self.candidate_refreshes += 1
        self.builder.assert_candidate_capacity()
        self.launch()
        stats = self.read_stats()
        self.recovery_replays += 1
        if stats.capacity_overflow:
            self.integrator.restore()
            raise FixedCapacityOverflow(stats.max_edges, stats.max_triplets)
        if not stats.overflow:
            return
        self.integrator.restore()
        for _ in range(self.steps_per_launch):
            self.builder.refresh_candidates(self.integrator.positions)
            self.candidate_refreshes += 1
            self._step_body(last=True)
            stats = self._read_now()
            if stats.capacity_overflow:
                raise FixedCapacityOverflow(stats.max_edges, stats.max_triplets)
        _require_finite_displacement(stats.max_displacement, self.launches)

    def _read_now(self) -> WindowStats:
        s = self._window_stats.tolist()
        return WindowStats(bool(s[0]), int(s[1]), float(s[3]), bool(s[4]), int(s[5]), int(s[6]), int(s[2]))

    def replay(self) -> WindowStats:
        """One window: launch, read its statistics, settle."""
        self.launch()
        stats = self.read_stats()
        self.settle(stats)
        return stats

    def stats(self) -> dict:
        """whole_step_cuda_graph.py:724-736."""
        return {
            "launches": self.launches,
            "steps_per_launch": self.steps_per_launch,
            "candidate_refreshes": self.candidate_refreshes,
            "fallback_windows": self.fallback_windows,
            "recovery_replays": self.recovery_replays,
            "max_edge_count": self.max_edge_count,
            "last_edge_count": self.last_edge_count,
            "max_displacement": self.max_displacement_seen,
            "e_capacity": self.builder.e_capacity,
            "warmup_runs": self.warmup_runs,
        }
