"""Asynchronous trajectory / log writer of the GPU-resident MD (fastmd/execution/gpu_logging.py:38-355).

The MD loop enqueues non-blocking device -> pinned-host copies into a ring of frame slots on a
copy stream; a writer thread waits on each slot's event and does the file I/O, so the MD stream
never waits for the host. A writer failure is recorded, later frames are dropped (their slots
still released), and the next ``enqueue`` / ``flush`` / ``close`` in the calling thread raises it.

The reference writes ASE ``Trajectory`` objects; ASE is not a dependency here, so a trajectory is
an object with ``write(frame)`` (``md_protocol.ExtxyzTrajectory``, or a path ending in ``.xyz`` /
``.extxyz``), and a frame is a :class:`Frame` (the fields an ASE ``Atoms`` with a single-point
calculator carries). The text log keeps the reference's header and format.
"""
from __future__ import annotations

import queue
import sys
import threading
from dataclasses import dataclass, field
from pathlib import Path
from typing import IO

import numpy as np
import torch
from torch import Tensor


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

    @property
    def velocities(self) -> np.ndarray:
        return self.momenta / self.masses[:, None]


@dataclass
class AtomsTemplate:
    """Numbers, masses, cell and pbc of the logged system (the reference's ``atoms_template``)."""

    numbers: np.ndarray
    masses: np.ndarray
    cell: np.ndarray
    pbc: np.ndarray

    def __len__(self) -> int:
        return int(len(self.numbers))

    @classmethod
    def of(cls, atoms) -> "AtomsTemplate":
        if isinstance(atoms, AtomsTemplate):
            return atoms
        if hasattr(atoms, "get_atomic_numbers"):
            cell = getattr(atoms.get_cell(), "array", atoms.get_cell())
            pbc = atoms.get_pbc() if hasattr(atoms, "get_pbc") else np.ones(3, bool)
            return cls(np.asarray(atoms.get_atomic_numbers()), np.asarray(atoms.get_masses(), np.float64),
                       np.asarray(cell, np.float64), np.asarray(pbc, bool))
        return cls(np.asarray(atoms.numbers), np.asarray(atoms.masses, np.float64), np.asarray(atoms.cell, np.float64),
                   np.asarray(getattr(atoms, "pbc", np.ones(3, bool)), bool))


@dataclass
class _FrameSlot:
    positions: Tensor
    momenta: Tensor
    forces: Tensor
    cell: Tensor
    scalars: Tensor
    extras: dict
    stress: Tensor | None = None
    event: torch.cuda.Event | None = None


@dataclass
class _PendingFrame:
    slot: _FrameSlot
    step: int
    time_ps: float


class AsyncGPUMDLogger:
    """Asynchronous trajectory/log writer (gpu_logging.py:38-355): same arguments and methods."""

    def __init__(self, atoms_template, device: torch.device, trajectory=None, logfile: str | Path | IO[str] | None = None,
                 loginterval: int = 1, append_trajectory: bool = False, ring: int = 8,
                 state_dtype: torch.dtype = torch.float32, extras: dict[str, int] | None = None, stress: bool = False,
                 value_dtype: torch.dtype = torch.float32) -> None:
        self.enabled = trajectory is not None or logfile is not None
        self.state_dtype = state_dtype
        self.extras = dict(extras or {})
        self.stress = bool(stress)
        self.loginterval = max(int(loginterval), 1)
        self.device = torch.device(device)
        self.atoms_template = AtomsTemplate.of(atoms_template)
        self._stop = object()
        self._available: queue.Queue = queue.Queue(maxsize=max(int(ring), 1))
        self._pending: queue.Queue = queue.Queue()
        self._thread: threading.Thread | None = None
        self._traj = None
        self._close_traj = False
        self._log = None
        self._close_log = False
        self._failure: tuple[int, BaseException] | None = None
        self._failure_reported = False
        self._stream = None
        if not self.enabled:
            return
        if trajectory is not None:
            if isinstance(trajectory, (str, Path)):
                suffix = Path(trajectory).suffix.lower()
                if suffix not in (".xyz", ".extxyz"):
                    raise ValueError(f"trajectory {trajectory}: this build writes EXTXYZ (.xyz / .extxyz) frames; "
                                     "ASE's binary .traj format needs ASE")
                from fastmd_amd.execution.md_protocol import ExtxyzTrajectory

                self._traj = ExtxyzTrajectory(trajectory, append=append_trajectory)
                self._close_traj = True
            else:
                self._traj = trajectory
        if logfile is not None:
            if logfile == "-":
                self._log = sys.stdout
            elif isinstance(logfile, (str, Path)):
                self._log = open(logfile, "a", encoding="utf-8")
                self._close_log = True
            else:
                self._log = logfile
            self._write_log_header()
        pin = self.device.type == "cuda"
        n = len(self.atoms_template)
        for _ in range(max(int(ring), 1)):
            self._available.put(_FrameSlot(
                positions=torch.empty((n, 3), dtype=state_dtype, pin_memory=pin),
                momenta=torch.empty((n, 3), dtype=state_dtype, pin_memory=pin),
                forces=torch.empty((n, 3), dtype=value_dtype, pin_memory=pin),
                cell=torch.empty((3, 3), dtype=value_dtype, pin_memory=pin),
                scalars=torch.empty((4,), dtype=torch.float64, pin_memory=pin),
                extras={name: torch.empty((int(size),), dtype=torch.float64, pin_memory=pin)
                        for name, size in self.extras.items()},
                stress=torch.empty((3, 3), dtype=value_dtype, pin_memory=pin) if self.stress else None))
        self._stream = torch.cuda.Stream(device=self.device) if pin else None
        self._thread = threading.Thread(target=self._writer_loop, daemon=True)
        self._thread.start()

    def _write_log_header(self) -> None:
        n = len(self.atoms_template)
        self._log_digits = 4 if n <= 100 else 3 if n <= 1000 else 2 if n <= 10000 else 1
        self._log.write("%-9s %12s %12s %12s  %6s\n" % ("Time[ps]", "Etot[eV]", "Epot[eV]", "Ekin[eV]", "T[K]"))
        self._log.flush()

    def should_log(self, step: int) -> bool:
        return self.enabled and step % self.loginterval == 0

    @property
    def copy_stream(self):
        """The stream of the device-to-host copies (None on a CPU device or without outputs)."""
        return self._stream

    def enqueue(self, *, step: int, time_ps: float, positions: Tensor, momenta: Tensor, forces: Tensor, cell: Tensor,
                potential_energy: Tensor, kinetic_energy: Tensor, temperature: Tensor, extras: dict | None = None,
                stress: Tensor | None = None) -> None:
        if not self.enabled:
            return
        self._raise_writer_failure()
        extras = extras or {}
        if set(extras) != set(self.extras):
            raise ValueError(f"logger extras {sorted(self.extras)} != enqueued {sorted(extras)}")
        if (stress is not None) != self.stress:
            raise ValueError(f"logger stress={self.stress}, but the enqueued frame "
                             f"{'has' if stress is not None else 'has no'} stress")
        slot = self._available.get()
        dev = positions.device
        scalars = torch.stack([torch.as_tensor(v, device=dev).reshape(()).to(torch.float64)
                               for v in (potential_energy, kinetic_energy, temperature)]
                              + [torch.zeros((), dtype=torch.float64, device=dev)])
        if self._stream is None:
            slot.positions.copy_(positions.detach().cpu())
            slot.momenta.copy_(momenta.detach().cpu())
            slot.forces.copy_(forces.detach().cpu())
            slot.cell.copy_(cell.detach().cpu())
            slot.scalars.copy_(scalars.detach().cpu())
            for name, value in extras.items():
                slot.extras[name].copy_(torch.as_tensor(value).detach().reshape(-1).cpu())
            if stress is not None:
                slot.stress.copy_(stress.detach().reshape(3, 3).cpu())
            slot.event = None
        else:
            producer = torch.cuda.current_stream(self.device)
            self._stream.wait_stream(producer)
            with torch.cuda.stream(self._stream):
                slot.positions.copy_(positions.detach(), non_blocking=True)
                slot.momenta.copy_(momenta.detach(), non_blocking=True)
                slot.forces.copy_(forces.detach(), non_blocking=True)
                slot.cell.copy_(cell.detach(), non_blocking=True)
                slot.scalars.copy_(scalars, non_blocking=True)
                for name, value in extras.items():
                    slot.extras[name].copy_(torch.as_tensor(value, device=dev).detach().reshape(-1),
                                            non_blocking=True)
                if stress is not None:
                    slot.stress.copy_(stress.detach().reshape(3, 3), non_blocking=True)
                slot.event = torch.cuda.Event()
                slot.event.record(self._stream)
            # write-after-read guard: later producer work (the next window overwrites the state
            # in place) waits for the copy; the host never blocks
            producer.wait_event(slot.event)
        self._pending.put(_PendingFrame(slot=slot, step=int(step), time_ps=float(time_ps)))

    def _writer_loop(self) -> None:
        while True:
            item = self._pending.get()
            if item is self._stop:
                self._pending.task_done()
                return
            try:
                if self._failure is None:
                    if item.slot.event is not None:
                        item.slot.event.synchronize()
                    self._write_frame(item)
            except BaseException as exc:  # noqa: BLE001 - re-raised in the caller's thread
                self._failure = (item.step, exc)
            finally:
                self._available.put(item.slot)
                self._pending.task_done()

    def _raise_writer_failure(self) -> None:
        failure = self._failure
        if failure is None:
            return
        step, exc = failure
        self._failure_reported = True
        detail = str(exc).strip().splitlines()
        raise RuntimeError(f"AsyncGPUMDLogger writer thread failed on the frame of step {step} "
                           f"({type(exc).__name__}: {detail[0] if detail else ''}); "
                           "the trajectory/log is incomplete from that frame on") from exc

    def _write_frame(self, frame: _PendingFrame) -> None:
        scalars = frame.slot.scalars.numpy()
        epot, ekin, temp = float(scalars[0]), float(scalars[1]), float(scalars[2])
        if self._traj is not None:
            t = self.atoms_template
            self._traj.write(Frame(
                numbers=t.numbers, masses=t.masses, cell=np.array(frame.slot.cell.numpy(), dtype=np.float64),
                pbc=t.pbc, positions=np.array(frame.slot.positions.numpy(), dtype=np.float64),
                momenta=np.array(frame.slot.momenta.numpy(), dtype=np.float64),
                forces=np.array(frame.slot.forces.numpy(), dtype=np.float64), energy=epot,
                info={name: np.array(value.numpy(), copy=True) for name, value in frame.slot.extras.items()},
                stress=None if frame.slot.stress is None else np.array(frame.slot.stress.numpy(), dtype=np.float64)))
        if self._log is not None:
            digits = getattr(self, "_log_digits", 3)
            fmt = "%-10.4f " + 3 * (f"%12.{digits}f ") + " %6.1f\n"
            self._log.write(fmt % (frame.time_ps, epot + ekin, epot, ekin, temp))
            self._log.flush()
        # a non-finite state on values already on the host (no extra sync)
        bad = int((~np.isfinite(frame.slot.positions.numpy()).all(axis=1)).sum())
        if bad or not np.isfinite(scalars[:3]).all():
            raise ValueError(f"non-finite MD state (frame written): Epot={epot}, Ekin={ekin}, T={temp}, "
                             f"{bad} atoms with non-finite positions")

    def flush(self) -> None:
        if not self.enabled:
            return
        self._pending.join()
        self._raise_writer_failure()

    def close(self) -> None:
        if not self.enabled:
            return
        self._pending.join()
        self._pending.put(self._stop)
        if self._thread is not None:
            self._thread.join()
            self._thread = None
        if self._traj is not None and self._close_traj:
            self._traj.close()
        if self._log is not None and self._close_log:
            self._log.close()
        self.enabled = False
        if not self._failure_reported:
            self._raise_writer_failure()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass
