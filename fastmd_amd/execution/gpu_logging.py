"""Asynchronous trajectory / log writer of the GPU-resident MD.

Replaces ``AsyncGPUMDLogger`` (fastmd/execution/gpu_logging.py:38-355) with the same constructor
arguments and methods (``should_log``, ``enqueue``, ``flush``, ``close``, ``copy_stream``).

Design. A fixed ring of pinned host staging slots, one per frame in flight. ``enqueue`` takes a
free slot, issues the device -> host copies on a dedicated copy stream that first waits for the
MD stream, records an event, and makes the MD stream wait for that event (the next window may
overwrite the state in place only after the copy has read it; the host never blocks). It then
hands the slot to a single-worker executor: the worker waits on the slot's event, formats the
frame and the text-log line, and returns. Each submission is a future; a slot returns to the
ring when its future is collected, oldest first, so frames are written in order and a full ring
makes ``enqueue`` wait for the oldest frame only. A worker error marks the logger broken: later
frames are skipped (their slots still recycled) and the error is raised once in the caller's
thread, at the next ``enqueue`` / ``flush`` / ``close``.

ASE is not a dependency: a trajectory is an object with ``write(frame)`` (``md_protocol.
ExtxyzTrajectory``, or a path ending in ``.xyz`` / ``.extxyz``), a frame a :class:`Frame`. The text
log keeps the reference's format: header ``Time[ps] Etot[eV] Epot[eV] Ekin[eV] T[K]`` and one row
per frame, energies with 4 / 3 / 2 / 1 decimals up to 100 / 1 000 / 10 000 / more atoms.
"""
from __future__ import annotations

import sys
import threading
from collections import deque
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass, field
from pathlib import Path
from typing import IO

import numpy as np
import torch
from torch import Tensor

from fastmd_amd._roctx import roctx_ranged


@dataclass
class Frame:
    """One logged MD frame on the host (what the reference's Atoms + calculator hold)."""

    numbers: np.ndarray
    masses: np.ndarray
    cell: np.ndarray
    pbc: np.ndarray
    positions: np.ndarray
    momenta: np.ndarray
    forces: np.ndarray
    energy: float
    info: dict = field(default_factory=dict)
    stress: np.ndarray | None = None
    explicit_masses: bool = False

    @property
    def velocities(self) -> np.ndarray:
        return self.momenta / self.masses[:, None]


@dataclass
class AtomsTemplate:
    """Numbers, masses, cell and pbc of the logged system (the reference's ``atoms_template``).
    ``explicit_masses``: the masses were given per atom (an ASE ``Atoms`` holding a ``masses``
    array), so frames carry a masses column as ASE's EXTXYZ writer does for such atoms."""

    numbers: np.ndarray
    masses: np.ndarray
    cell: np.ndarray
    pbc: np.ndarray
    explicit_masses: bool = False

    def __len__(self) -> int:
        return int(len(self.numbers))

    @classmethod
    def of(cls, atoms) -> "AtomsTemplate":
        if isinstance(atoms, AtomsTemplate):
            return atoms
        if hasattr(atoms, "get_atomic_numbers"):
            cell = getattr(atoms.get_cell(), "array", atoms.get_cell())
            pbc = atoms.get_pbc() if hasattr(atoms, "get_pbc") else np.ones(3, bool)
            explicit = "masses" in getattr(atoms, "arrays", {})
            return cls(np.asarray(atoms.get_atomic_numbers()), np.asarray(atoms.get_masses(), np.float64),
                       np.asarray(cell, np.float64), np.asarray(pbc, bool), explicit)
        return cls(np.asarray(atoms.numbers), np.asarray(atoms.masses, np.float64), np.asarray(atoms.cell, np.float64),
                   np.asarray(getattr(atoms, "pbc", np.ones(3, bool)), bool), True)


def log_decimals(n_atoms: int) -> int:
    """Decimals of the text log's energy columns (the reference's thresholds)."""
    for limit, digits in ((100, 4), (1000, 3), (10000, 2)):
        if n_atoms <= limit:
            return digits
    return 1


LOG_HEADER = "%-9s %12s %12s %12s  %6s\n" % ("Time[ps]", "Etot[eV]", "Epot[eV]", "Ekin[eV]", "T[K]")


def log_row(time_ps: float, epot: float, ekin: float, temperature: float, digits: int) -> str:
    return ("%-10.4f " + 3 * f"%12.{digits}f " + " %6.1f\n") % (time_ps, epot + ekin, epot, ekin, temperature)


class _Staging:
    """Pinned host buffers of one frame in flight: the state rows, the cell, (Epot, Ekin, T), the
    extras and the stress, plus the event that marks the end of their copies."""

    def __init__(self, n: int, state_dtype, value_dtype, extras: dict, stress: bool, pin: bool) -> None:
        new = lambda shape, dtype: torch.empty(shape, dtype=dtype, pin_memory=pin)  # noqa: E731
        self.positions = new((n, 3), state_dtype)
        self.momenta = new((n, 3), state_dtype)
        self.forces = new((n, 3), value_dtype)
        self.cell = new((3, 3), value_dtype)
        self.energies = new((3,), torch.float64)
        self.extras = {name: new((int(size),), torch.float64) for name, size in extras.items()}
        self.stress = new((3, 3), value_dtype) if stress else None
        self.ready: torch.cuda.Event | None = None

    def fill(self, source: dict, copy_stream) -> None:
        """Copy every field of ``source`` (device or host tensors) into the slot; on a device,
        asynchronously on ``copy_stream`` with ``ready`` recorded after the last copy."""
        if copy_stream is None:
            for name, value in source.items():
                self._target(name).copy_(value.detach().reshape(self._target(name).shape).cpu())
            self.ready = None
            return
        with torch.cuda.stream(copy_stream):
            for name, value in source.items():
                dst = self._target(name)
                dst.copy_(value.detach().reshape(dst.shape), non_blocking=True)
            self.ready = torch.cuda.Event()
            self.ready.record(copy_stream)

    def _target(self, name: str) -> Tensor:
        if name.startswith("extra:"):
            return self.extras[name[6:]]
        return getattr(self, name)


class AsyncGPUMDLogger:
    """Asynchronous trajectory / text-log writer (the reference's arguments and methods)."""

    def __init__(self, atoms_template, device: torch.device, trajectory=None, logfile: str | Path | IO[str] | None = None,
                 loginterval: int = 1, append_trajectory: bool = False, ring: int = 8,
                 state_dtype: torch.dtype = torch.float32, extras: dict[str, int] | None = None, stress: bool = False,
                 value_dtype: torch.dtype = torch.float32) -> None:
        self.atoms_template = AtomsTemplate.of(atoms_template)
        self.device = torch.device(device)
        self.loginterval = max(int(loginterval), 1)
        self.state_dtype = state_dtype
        self.extras = dict(extras or {})
        self.stress = bool(stress)
        self.enabled = trajectory is not None or logfile is not None
        self._owned: list = []  # files this logger opened and closes
        self._trajectory = self._open_trajectory(trajectory, append_trajectory)
        self._log = self._open_log(logfile)
        self._digits = log_decimals(len(self.atoms_template))
        self._broken = threading.Event()  # set by the worker on its first failure
        self._failure: tuple[int, BaseException] | None = None
        self._reported = False
        self._free: deque[_Staging] = deque()
        self._in_flight: deque[tuple[Future, _Staging, int]] = deque()
        self._worker: ThreadPoolExecutor | None = None
        self._copies = None
        if not self.enabled:
            return
        if self._log is not None:
            self._log.write(LOG_HEADER)
            self._log.flush()
        on_gpu = self.device.type == "cuda"
        n = len(self.atoms_template)
        self._free.extend(_Staging(n, state_dtype, value_dtype, self.extras, self.stress, on_gpu)
                          for _ in range(max(int(ring), 1)))
        self._copies = torch.cuda.Stream(device=self.device) if on_gpu else None
        self._worker = ThreadPoolExecutor(max_workers=1, thread_name_prefix="fastmd-frame-writer")

    # ------------------------------------------------------------------ files
    def _open_trajectory(self, trajectory, append: bool):
        if trajectory is None or not isinstance(trajectory, (str, Path)):
            return trajectory
        if Path(trajectory).suffix.lower() not in (".xyz", ".extxyz"):
            raise ValueError(f"trajectory {trajectory}: frames are written as EXTXYZ (.xyz / .extxyz); "
                             "the binary .traj format is ASE's and ASE is not used here")
        from fastmd_amd.execution.md_protocol import ExtxyzTrajectory

        stream = ExtxyzTrajectory(trajectory, append=append)
        self._owned.append(stream)
        return stream

    def _open_log(self, logfile):
        if logfile is None or logfile == "-":
            return None if logfile is None else sys.stdout
        if isinstance(logfile, (str, Path)):
            stream = open(logfile, "a", encoding="utf-8")
            self._owned.append(stream)
            return stream
        return logfile

    # ------------------------------------------------------------------ public API
    @property
    def copy_stream(self):
        """The stream of the device-to-host copies (None on a CPU device or without outputs)."""
        return self._copies

    def should_log(self, step: int) -> bool:
        return self.enabled and step % self.loginterval == 0

    @roctx_ranged("logger enqueue")
    def enqueue(self, *, step: int, time_ps: float, positions: Tensor, momenta: Tensor, forces: Tensor, cell: Tensor,
                potential_energy: Tensor, kinetic_energy: Tensor, temperature: Tensor, extras: dict | None = None,
                stress: Tensor | None = None) -> None:
        """Stage one frame (asynchronous copies) and queue its file writes."""
        if not self.enabled:
            return
        self._raise_failure()
        extras = extras or {}
        if extras.keys() != self.extras.keys():
            raise ValueError(f"frame extras {sorted(extras)} differ from the logger's {sorted(self.extras)}")
        if self.stress != (stress is not None):
            raise ValueError("the frame's stress does not match the logger's stress setting "
                             f"(logger stress={self.stress})")
        dev = positions.device
        energies = torch.stack([torch.as_tensor(v, device=dev).reshape(()).to(torch.float64)
                                for v in (potential_energy, kinetic_energy, temperature)])
        source = {"positions": positions, "momenta": momenta, "forces": forces, "cell": cell, "energies": energies}
        source.update({f"extra:{k}": torch.as_tensor(v, device=dev) for k, v in extras.items()})
        if stress is not None:
            source["stress"] = stress
        slot = self._take_slot()
        if self._copies is not None:
            md_stream = torch.cuda.current_stream(self.device)
            self._copies.wait_stream(md_stream)
            slot.fill(source, self._copies)
            md_stream.wait_event(slot.ready)  # the MD may overwrite the state only after the copy
        else:
            slot.fill(source, None)
        future = self._worker.submit(self._emit, slot, int(step), float(time_ps))
        self._in_flight.append((future, slot, int(step)))

    def flush(self) -> None:
        """Wait until every queued frame is written; raise a writer failure."""
        if not self.enabled:
            return
        self._collect(until_empty=True)
        self._raise_failure()

    def close(self) -> None:
        """Write what is queued, stop the worker, close the files this logger opened; raise a
        writer failure that was not raised before."""
        if not self.enabled:
            return
        self.enabled = False
        try:
            self._collect(until_empty=True)
        finally:
            self._worker.shutdown(wait=True)
            for stream in self._owned:
                stream.close()
            self._owned.clear()
        if not self._reported:
            self._raise_failure()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    # ------------------------------------------------------------------ ring
    def _take_slot(self) -> _Staging:
        self._collect(until_empty=False)
        if not self._free:  # ring full: wait for the oldest frame
            self._collect_one()
        return self._free.popleft()

    def _collect(self, until_empty: bool) -> None:
        while self._in_flight and (until_empty or self._in_flight[0][0].done()):
            self._collect_one()

    def _collect_one(self) -> None:
        future, slot, step = self._in_flight.popleft()
        error = future.exception()
        if error is not None and self._failure is None:
            self._failure = (step, error)
        self._free.append(slot)

    def _raise_failure(self) -> None:
        if self._failure is None:
            return
        step, error = self._failure
        self._reported = True
        first = (str(error).strip().splitlines() or [""])[0]
        raise RuntimeError(f"trajectory/log writer stopped at the frame of step {step} "
                           f"({type(error).__name__}: {first}); later frames were not written") from error

    # ------------------------------------------------------------------ worker thread
    def _emit(self, slot: _Staging, step: int, time_ps: float) -> None:
        if self._broken.is_set():
            return
        try:
            if slot.ready is not None:
                slot.ready.synchronize()
            epot, ekin, temperature = (float(x) for x in slot.energies.numpy())
            positions = np.array(slot.positions.numpy(), dtype=np.float64)
            if self._trajectory is not None:
                t = self.atoms_template
                self._trajectory.write(Frame(
                    numbers=t.numbers, masses=t.masses, cell=np.array(slot.cell.numpy(), dtype=np.float64), pbc=t.pbc,
                    positions=positions, momenta=np.array(slot.momenta.numpy(), dtype=np.float64),
                    forces=np.array(slot.forces.numpy(), dtype=np.float64), energy=epot,
                    info={name: np.array(v.numpy(), copy=True) for name, v in slot.extras.items()},
                    stress=None if slot.stress is None else np.array(slot.stress.numpy(), dtype=np.float64),
                    explicit_masses=t.explicit_masses))
            if self._log is not None:
                self._log.write(log_row(time_ps, epot, ekin, temperature, self._digits))
                self._log.flush()
            finite_rows = np.isfinite(positions).all(axis=1)
            if not finite_rows.all() or not np.isfinite([epot, ekin, temperature]).all():
                raise ValueError(f"the MD state is not finite (the frame was written): {int((~finite_rows).sum())} "
                                 f"atoms with non-finite positions, Epot={epot}, Ekin={ekin}, T={temperature}")
        except BaseException:
            self._broken.set()
            raise
