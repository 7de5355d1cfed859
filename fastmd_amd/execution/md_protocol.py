"""MD output files and the restart file (fastmd/execution/md_protocol.py:1-447).

Formats kept from the reference: the thermo text (``THERMO_HEADER`` columns, tab separated),
EXTXYZ frames with velocities, energy, forces and the logger's per-frame extras as scalar or
vector ``info`` entries, and the ID-ordered restart ``.npz`` (``RESTART_FORMAT``
"fastmd.distributed.md/1", the same keys) that records the other files' sizes so that a resume
truncates them to the checkpoint. ``MDOutputs`` is the single-process form of the reference's
(one GPU: every "gather by ID" is the identity, ids = arange(N)).
"""
from __future__ import annotations

import json
import math
import os
import weakref
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

THERMO_FILE, TRAJECTORY_FILE, RESTART_FILE = "md_thermo.txt", "md_trajectory.extxyz", "md_restart.npz"
THERMO_HEADER = ("# Step\tTime(fs)\tTargetTemperature(K)\tTemperature(K)\t"
                 "PotentialEnergy(eV)\tKineticEnergy(eV)\tTotalEnergy(eV)\n")
RESTART_FORMAT = "fastmd.distributed.md/1"
_ERRORS = (TypeError, ValueError, RuntimeError, AttributeError, IndexError, KeyError)

_SYMBOLS = (
    "X H He Li Be B C N O F Ne Na Mg Al Si P S Cl Ar K Ca Sc Ti V Cr Mn Fe Co Ni Cu Zn Ga Ge As Se Br Kr "
    "Rb Sr Y Zr Nb Mo Tc Ru Rh Pd Ag Cd In Sn Sb Te I Xe Cs Ba La Ce Pr Nd Pm Sm Eu Gd Tb Dy Ho Er Tm Yb "
    "Lu Hf Ta W Re Os Ir Pt Au Hg Tl Pb Bi Po At Rn Fr Ra Ac Th Pa U Np Pu Am Cm Bk Cf Es Fm Md No Lr Rf "
    "Db Sg Bh Hs Mt Ds Rg Cn Nh Fl Mc Lv Ts Og").split()


def chemical_symbol(z: int) -> str:
    return _SYMBOLS[int(z)]


def _info_value(key: str, value) -> str:
    arr = np.asarray(value).reshape(-1)
    if arr.size == 1:
        v = arr[0]
        if key == "step":
            return str(int(v))
        return repr(float(v))
    return '"' + " ".join(repr(float(v)) for v in arr) + '"'


class ExtxyzTrajectory:
    """Truncatable EXTXYZ trajectory (md_protocol.py:90-118): frames carry velocities (momenta /
    masses), energy and forces; scalar extras as numbers (``step`` an integer), vector extras
    quoted. Every frame is flushed, so after ``logger.flush()`` the file size is a frame boundary
    (the offset a restart records)."""

    def __init__(self, path, *, append: bool):
        self._stream = open(path, "a" if append else "w", encoding="utf-8")

    def write(self, frame) -> None:
        cell = np.asarray(frame.cell, np.float64).reshape(3, 3)
        lattice = " ".join(repr(float(v)) for v in cell.reshape(-1))
        pbc = " ".join("T" if p else "F" for p in np.asarray(frame.pbc, bool).reshape(3))
        info = "".join(f" {k}={_info_value(k, v)}" for k, v in frame.info.items())
        head = (f'Lattice="{lattice}" Properties=species:S:1:pos:R:3:velocities:R:3:forces:R:3 '
                f"energy={float(frame.energy)!r}{info} pbc=\"{pbc}\"")
        vel = frame.velocities
        lines = [str(len(frame.numbers)), head]
        for z, p, v, f in zip(frame.numbers, frame.positions, vel, frame.forces):
            lines.append(f"{chemical_symbol(z):<2s} " + " ".join(f"{x:16.8f}" for x in (*p, *v, *f)))
        self._stream.write("\n".join(lines) + "\n")
        self._stream.flush()

    def close(self) -> None:
        self._stream.close()


def read_extxyz(path) -> list[dict]:
    """The frames an :class:`ExtxyzTrajectory` wrote: symbols, positions, velocities, forces,
    cell, pbc, energy and the info entries (host numpy)."""
    frames = []
    with open(path, encoding="utf-8") as stream:
        lines = stream.read().splitlines()
    i = 0
    while i < len(lines):
        n = int(lines[i])
        head = lines[i + 1]
        info, key, j = {}, None, 0
        tokens = []
        while j < len(head):  # key=value pairs, values possibly quoted
            eq = head.index("=", j)
            key = head[j:eq].strip()
            if head[eq + 1] == '"':
                end = head.index('"', eq + 2)
                value, j = head[eq + 2:end], end + 1
            else:
                end = head.find(" ", eq + 1)
                end = len(head) if end < 0 else end
                value, j = head[eq + 1:end], end
            tokens.append((key, value))
            while j < len(head) and head[j] == " ":
                j += 1
        for key, value in tokens:
            info[key] = value
        rows = [line.split() for line in lines[i + 2:i + 2 + n]]
        data = np.array([[float(x) for x in r[1:]] for r in rows], np.float64).reshape(n, 9)
        extra = {k: (int(v) if k == "step" else np.array([float(x) for x in v.split()]) if " " in v else float(v))
                 for k, v in info.items() if k not in ("Lattice", "Properties", "pbc", "energy")}
        frames.append({"symbols": [r[0] for r in rows], "positions": data[:, 0:3], "velocities": data[:, 3:6],
                       "forces": data[:, 6:9], "cell": np.array([float(x) for x in info["Lattice"].split()]).reshape(3, 3),
                       "pbc": np.array([t == "T" for t in info["pbc"].split()]), "energy": float(info["energy"]),
                       "info": extra})
        i += 2 + n
    return frames


@dataclass
class RestartData:
    """One restart file as host (numpy) arrays, rows in ID order (md_protocol.py:121-149)."""

    ids: np.ndarray
    numbers: np.ndarray
    masses: np.ndarray
    positions: np.ndarray
    momenta: np.ndarray
    forces: np.ndarray
    energy: np.ndarray
    reference_energy: np.ndarray
    cell: np.ndarray
    pbc: np.ndarray
    step: int
    parameters: dict
    temperature_K: float | None
    nhc_state: dict | None
    offsets: dict
    engine: str


def read_restart(path) -> RestartData:
    """Parse a :func:`write_restart` file (md_protocol.py:152-174)."""
    with np.load(path) as data:
        if str(data["format"]) != RESTART_FORMAT:
            raise ValueError(f"not a {RESTART_FORMAT} restart file")
        parameters = json.loads(str(data["parameters"]))
        temperature = float(data["temperature_K"])
        nhc = parameters["ensemble"] == "nvt_nhc"
        return RestartData(
            ids=data["ids"], numbers=data["numbers"], masses=data["masses"], positions=data["positions"],
            momenta=data["momenta"], forces=data["forces"], energy=data["potential_energy"],
            reference_energy=data["reference_energy"], cell=data["cell"], pbc=data["pbc"], step=int(data["step"]),
            parameters=parameters, temperature_K=None if math.isnan(temperature) else temperature,
            nhc_state={"temperature_K": temperature, "eta": np.array(data["nhc_eta"]),
                       "p_eta": np.array(data["nhc_p_eta"])} if nhc else None,
            offsets=json.loads(str(data["offsets"])),
            engine=str(data["engine"]) if "engine" in data.files else "domain")


def write_restart(path, data: RestartData) -> None:
    """Write ``data`` atomically (temporary file + os.replace) as an ``.npz`` (md_protocol.py:177-190)."""
    path = Path(path)
    nhc = {} if data.nhc_state is None else data.nhc_state
    temporary = path.with_name(path.name + ".tmp.npz")
    np.savez(temporary, format=np.array(RESTART_FORMAT), ids=data.ids, numbers=data.numbers, masses=data.masses,
             positions=data.positions, momenta=data.momenta, forces=data.forces, potential_energy=data.energy,
             reference_energy=data.reference_energy, cell=data.cell, pbc=data.pbc,
             step=np.array(data.step, dtype=np.int64), parameters=np.array(json.dumps(data.parameters)),
             temperature_K=np.array(math.nan if data.temperature_K is None else data.temperature_K),
             nhc_eta=nhc.get("eta", np.zeros(0)), nhc_p_eta=nhc.get("p_eta", np.zeros(0)),
             offsets=np.array(json.dumps(data.offsets)), engine=np.array(data.engine))
    os.replace(temporary, path)


def resume_mismatch(saved: dict, requested: dict, *, ignore=()) -> dict:
    """``{key: (saved, requested)}`` for every parameter a continuation changes (md_protocol.py:193-202)."""
    skip = {"total_steps", *ignore}
    return {key: (saved.get(key), requested.get(key)) for key in sorted(saved.keys() | requested.keys())
            if key not in skip and saved.get(key) != requested.get(key)}


class MDOutputs:
    """A driver's output files (md_protocol.py:205-447), one process: thermo line every
    ``thermo_interval`` steps, EXTXYZ frame every ``xyz_interval``, restart every
    ``restart_interval`` (0 disables each; ``output_dir`` None disables all), the last step
    (``total_steps``) always with a thermo line and a restart. A fresh start removes earlier
    outputs and writes the frame and restart of step 0; a resume passes the restart's ``offsets``
    and the files are truncated to them.

    ``source`` provides ``nsteps``, ``parameters``, ``cell``, ``device``, ``md_fields()``,
    ``thermodynamics()`` and ``thermostat_state()``."""

    def __init__(self, source, output_dir, thermo_interval: int, xyz_interval: int, restart_interval: int,
                 total_steps: int | None, offsets: dict | None, *, engine: str = "native"):
        self.source, self.engine = weakref.proxy(source), engine
        self.output_dir = None if output_dir is None else Path(output_dir)
        self.thermo_interval, self.xyz_interval = int(thermo_interval), int(xyz_interval)
        self.restart_interval, self.total_steps = int(restart_interval), total_steps
        self.logger, self._tracked = None, {}
        if self.output_dir is None:
            return
        self._tracked = {name: self.output_dir / name for name in (THERMO_FILE, TRAJECTORY_FILE)}
        self.output_dir.mkdir(parents=True, exist_ok=True)
        if offsets is None:
            for path in (*self._tracked.values(), self.output_dir / RESTART_FILE):
                path.unlink(missing_ok=True)
            with open(self._tracked[THERMO_FILE], "w") as stream:
                stream.write(THERMO_HEADER)
        else:
            sizes = {name: int(offsets[name]) for name, path in self._tracked.items()
                     if name in offsets and path.exists()}
            short = [name for name, size in sizes.items() if self._tracked[name].stat().st_size < size]
            if short:
                raise ValueError(f"cannot resume: {short} shorter than the restart file's offsets")
            for name, size in sizes.items():
                with open(self._tracked[name], "r+b") as stream:
                    stream.truncate(size)
        if self.xyz_interval:
            self.logger = self._frame_logger(offsets is not None)
        if offsets is None and (self.xyz_interval or self.restart_interval):
            if self.xyz_interval:
                self.log_frame(None)
            if self.restart_interval:
                self.save_restart(None)

    def _frame_logger(self, append: bool):
        from fastmd_amd.execution.gpu_logging import AsyncGPUMDLogger, AtomsTemplate

        fields = self.source.md_fields()
        template = AtomsTemplate(numbers=fields["numbers"].cpu().numpy(), masses=fields["masses"].double().cpu().numpy(),
                                 cell=self.source.cell.detach().cpu().double().numpy(), pbc=np.ones(3, bool))
        extras = {"step": 1, "time_fs": 1, "target_temp_K": 1}
        tchain = int(self.source.parameters["tchain"])
        extras.update(nhc_eta=tchain, nhc_p_eta=tchain, nhc_conserved_energy=1)
        trajectory = ExtxyzTrajectory(self._tracked[TRAJECTORY_FILE], append=append)
        try:
            return AsyncGPUMDLogger(template, self.source.device, trajectory=trajectory,
                                    state_dtype=fields["positions"].dtype, extras=extras)
        except BaseException:
            trajectory.close()
            raise

    def due(self, step: int) -> bool:
        """Whether the step writes any output (the driver settles such windows on their own)."""
        if self.output_dir is None:
            return False
        last = self.total_steps is not None and step == self.total_steps
        return bool((self.thermo_interval and (step % self.thermo_interval == 0 or last))
                    or (self.xyz_interval and step % self.xyz_interval == 0)
                    or (self.restart_interval and (step % self.restart_interval == 0 or last)))

    def write(self) -> dict | None:
        """Thermo line, frame and restart file due at the current step (call after every step)."""
        if self.output_dir is None:
            return None
        step = self.source.nsteps
        last = self.total_steps is not None and step == self.total_steps
        thermo_due = bool(self.thermo_interval) and (step % self.thermo_interval == 0 or last)
        xyz_due = bool(self.xyz_interval) and step % self.xyz_interval == 0
        restart_due = bool(self.restart_interval) and (step % self.restart_interval == 0 or last)
        if not (thermo_due or xyz_due or restart_due):
            return None
        thermo = self.source.thermodynamics()
        if thermo_due:
            target = thermo["target_temperature"]
            with open(self._tracked[THERMO_FILE], "a") as stream:
                stream.write(f"{step:d}\t{thermo['time_fs']:.4f}\t"
                             f"{math.nan if target is None else target:.4f}\t{thermo['temperature']:.4f}\t"
                             f"{thermo['potential_energy']:.6f}\t{thermo['kinetic_energy']:.6f}\t"
                             f"{thermo['total_energy']:.6f}\n")
        if xyz_due:
            self.log_frame(thermo)
        if restart_due:
            self.save_restart(None)
        return thermo

    def log_frame(self, thermo: dict | None = None) -> None:
        """The current frame into the EXTXYZ logger (asynchronous file write)."""
        if self.output_dir is None or not self.xyz_interval:
            raise RuntimeError("log_frame needs output_dir and xyz_interval")
        thermo = self.source.thermodynamics() if thermo is None else thermo
        fields = self.source.md_fields()
        scalar = lambda value: torch.tensor([value], dtype=torch.float64)  # noqa: E731
        extras = {"step": scalar(thermo["step"]), "time_fs": scalar(thermo["time_fs"]),
                  "target_temp_K": scalar(thermo["target_temperature"]),
                  "nhc_eta": torch.tensor(thermo["eta"], dtype=torch.float64),
                  "nhc_p_eta": torch.tensor(thermo["p_eta"], dtype=torch.float64),
                  "nhc_conserved_energy": scalar(thermo["conserved_energy"])}
        self.logger.enqueue(step=thermo["step"], time_ps=thermo["time_fs"] / 1000.0, positions=fields["positions"],
                            momenta=fields["momenta"], forces=fields["forces"], cell=self.source.cell,
                            potential_energy=scalar(thermo["potential_energy"]),
                            kinetic_energy=scalar(thermo["kinetic_energy"]),
                            temperature=scalar(thermo["temperature"]), extras=extras)

    def save_restart(self, path=None) -> None:
        """Write the current state to the restart file (default ``output_dir``), with the thermostat
        state and the output files' offsets."""
        if path is None and self.output_dir is None:
            raise ValueError("save_restart needs a path (no output_dir)")
        fields = self.source.md_fields()
        thermostat = self.source.thermostat_state()
        path = self.output_dir / RESTART_FILE if path is None else Path(path)
        if self.logger is not None:
            self.logger.flush()
        offsets = {name: file.stat().st_size if file.exists() else 0 for name, file in self._tracked.items()}
        host = lambda value, dtype=None: (value if dtype is None else value.to(dtype)).detach().cpu().numpy()  # noqa: E731
        write_restart(path, RestartData(
            ids=host(fields["ids"], torch.int64), numbers=host(fields["numbers"], torch.int64),
            masses=host(fields["masses"], torch.float64), positions=host(fields["positions"], torch.float64),
            momenta=host(fields["momenta"], torch.float64), forces=host(fields["forces"]),
            energy=host(fields["energy"]), reference_energy=host(fields["reference_energy"]),
            cell=host(self.source.cell), pbc=np.ones(3, dtype=bool), step=self.source.nsteps,
            parameters=self.source.parameters, temperature_K=thermostat.get("temperature_K"),
            nhc_state=thermostat, offsets=offsets, engine=self.engine))

    def close(self) -> None:
        logger, self.logger = self.logger, None
        if logger is not None:
            logger.close()

    def close_quietly(self) -> None:
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass
