"""MD output files and the restart file.

Replaces fastmd/execution/md_protocol.py:90-447 for one process (one GPU: every "gather by ID"
of the reference is the identity, ids = arange(N)). What is kept from the reference is the on-disk
format, so that files move between the two:

* the file names ``md_thermo.txt``, ``md_trajectory.extxyz``, ``md_restart.npz``;
* the thermo text: ``THERMO_HEADER`` and tab-separated rows (step, time, target and current
  temperature with 4 decimals, energies with 6);
* EXTXYZ frames as ASE's extxyz writer lays out a frame with a single-point calculator
  (md_protocol.py:104-114): ``Lattice`` (the cell rows), ``Properties`` (species, pos, masses when
  the atoms carry explicit masses, velocities, forces), the info entries in insertion order
  (``step`` an integer, one-element arrays as numbers, longer ones quoted), then ``energy``, then
  ``pbc``; per-atom rows ``%-2s`` then ``%16.8f`` columns;
* the restart ``.npz``: format tag ``fastmd.distributed.md/1`` and its keys (:121-190), written
  atomically, recording the other files' sizes so that a resume truncates them to the checkpoint;
  ``resume_mismatch`` (:193-202).

``MDOutputs`` (the driver's file outputs) is organised around one schedule per output kind and a
table of tracked files.
"""
from __future__ import annotations

import json
import math
import os
import weakref
from dataclasses import dataclass, fields
from pathlib import Path

import numpy as np
import torch

THERMO_FILE, TRAJECTORY_FILE, RESTART_FILE = "md_thermo.txt", "md_trajectory.extxyz", "md_restart.npz"
THERMO_HEADER = ("# Step\tTime(fs)\tTargetTemperature(K)\tTemperature(K)\t"
                 "PotentialEnergy(eV)\tKineticEnergy(eV)\tTotalEnergy(eV)\n")
RESTART_FORMAT = "fastmd.distributed.md/1"

_SYMBOLS = (
    "X H He Li Be B C N O F Ne Na Mg Al Si P S Cl Ar K Ca Sc Ti V Cr Mn Fe Co Ni Cu Zn Ga Ge As Se Br Kr "
    "Rb Sr Y Zr Nb Mo Tc Ru Rh Pd Ag Cd In Sn Sb Te I Xe Cs Ba La Ce Pr Nd Pm Sm Eu Gd Tb Dy Ho Er Tm Yb "
    "Lu Hf Ta W Re Os Ir Pt Au Hg Tl Pb Bi Po At Rn Fr Ra Ac Th Pa U Np Pu Am Cm Bk Cf Es Fm Md No Lr Rf "
    "Db Sg Bh Hs Mt Ds Rg Cn Nh Fl Mc Lv Ts Og").split()


def chemical_symbol(z: int) -> str:
    return _SYMBOLS[int(z)]


def thermo_row(step: int, thermo: dict) -> str:
    target = thermo["target_temperature"]
    cols = (thermo["time_fs"], math.nan if target is None else target, thermo["temperature"])
    energies = (thermo["potential_energy"], thermo["kinetic_energy"], thermo["total_energy"])
    return "\t".join([str(int(step))] + [f"{v:.4f}" for v in cols] + [f"{v:.6f}" for v in energies]) + "\n"


# ------------------------------------------------------------------------------------ EXTXYZ
def _number(value) -> str:
    return repr(float(value))


def _info_text(key: str, value) -> str:
    flat = np.asarray(value).reshape(-1)
    if flat.size != 1:
        return '"' + " ".join(_number(v) for v in flat) + '"'
    return str(int(flat[0])) if key == "step" else _number(flat[0])


class ExtxyzTrajectory:
    """Truncatable EXTXYZ trajectory: frames carry velocities (momenta / masses), forces, the
    energy and the logger's extras. Each frame is flushed, so once the logger is flushed the file
    size is a frame boundary (the offset a restart records)."""

    def __init__(self, path, *, append: bool):
        self._stream = open(path, "a" if append else "w", encoding="utf-8")

    def write(self, frame) -> None:
        columns = [("species", "S", 1, [chemical_symbol(z) for z in frame.numbers]),
                   ("pos", "R", 3, np.asarray(frame.positions, np.float64))]
        if getattr(frame, "explicit_masses", False):
            columns.append(("masses", "R", 1, np.asarray(frame.masses, np.float64).reshape(-1, 1)))
        columns += [("velocities", "R", 3, frame.velocities), ("forces", "R", 3, np.asarray(frame.forces, np.float64))]
        header = {"Lattice": '"' + " ".join(_number(v) for v in np.asarray(frame.cell, np.float64).reshape(-1)) + '"',
                  "Properties": ":".join(f"{name}:{kind}:{width}" for name, kind, width, _ in columns)}
        header.update({key: _info_text(key, value) for key, value in frame.info.items()})
        header["energy"] = _number(frame.energy)
        header["pbc"] = '"' + " ".join("T" if p else "F" for p in np.asarray(frame.pbc, bool).reshape(3)) + '"'
        out = [f"{len(frame.numbers)}\n", " ".join(f"{k}={v}" for k, v in header.items()) + "\n"]
        numeric = np.concatenate([c[3] for c in columns[1:]], axis=1)
        row_format = "%-2s " + " ".join(["%16.8f"] * numeric.shape[1]) + "\n"
        out.extend(row_format % (symbol, *values) for symbol, values in zip(columns[0][3], numeric))
        self._stream.write("".join(out))
        self._stream.flush()

    def close(self) -> None:
        self._stream.close()


def _header_pairs(line: str) -> dict:
    """key=value pairs of an EXTXYZ comment line (values possibly double-quoted)."""
    pairs, pos = {}, 0
    while pos < len(line):
        if line[pos] == " ":
            pos += 1
            continue
        eq = line.index("=", pos)
        key = line[pos:eq]
        if line[eq + 1] == '"':
            end = line.index('"', eq + 2)
            pairs[key], pos = line[eq + 2:end], end + 1
        else:
            end = line.find(" ", eq + 1)
            end = len(line) if end < 0 else end
            pairs[key], pos = line[eq + 1:end], end
    return pairs


def read_extxyz(path) -> list[dict]:
    """The frames of an EXTXYZ file as host numpy: symbols, every Properties column by name
    (``positions`` for pos), cell, pbc, energy, the remaining header entries in ``info`` and the
    header's key order in ``keys``."""
    frames = []
    with open(path, encoding="utf-8") as stream:
        lines = stream.read().splitlines()
    at = 0
    while at < len(lines):
        n = int(lines[at])
        header = _header_pairs(lines[at + 1])
        rows = [line.split() for line in lines[at + 2:at + 2 + n]]
        spec = header["Properties"].split(":")
        frame, col = {"keys": list(header)}, 0
        for name, kind, width in zip(spec[0::3], spec[1::3], map(int, spec[2::3])):
            if kind == "S":
                frame["symbols"] = [r[col] for r in rows]
            else:
                values = np.array([[float(x) for x in r[col:col + width]] for r in rows], np.float64)
                frame["positions" if name == "pos" else name] = values if width > 1 else values.reshape(-1)
            col += width
        frame["cell"] = np.array([float(x) for x in header["Lattice"].split()]).reshape(3, 3)
        frame["pbc"] = np.array([t == "T" for t in header["pbc"].split()])
        frame["energy"] = float(header["energy"])
        frame["info"] = {k: (int(v) if k == "step" else np.array([float(x) for x in v.split()]) if " " in v else float(v))
                         for k, v in header.items() if k not in ("Lattice", "Properties", "pbc", "energy")}
        frames.append(frame)
        at += 2 + n
    return frames


# ------------------------------------------------------------------------------------ restart
@dataclass
class RestartData:
    """One restart file as host (numpy) arrays, rows in ID order (md_protocol.py:121-149).
    ``positions`` float64 for nvt_nhc; ``forces``, ``energy``, ``reference_energy`` the cached
    evaluation of that state; ``temperature_K`` the thermostat target (None for nve);
    ``nhc_state`` the NHC ``state_dict`` (nvt_nhc only); ``offsets`` the output files' sizes."""

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


# fields stored as plain arrays under their own name, and the three renamed / encoded ones
_ARRAY_FIELDS = ("ids", "numbers", "masses", "positions", "momenta", "forces", "reference_energy", "cell", "pbc")
_JSON_FIELDS = ("parameters", "offsets")


def _encode_restart(data: RestartData) -> dict:
    nhc = data.nhc_state or {}
    record = {"format": np.array(RESTART_FORMAT), "potential_energy": data.energy,
              "step": np.array(data.step, dtype=np.int64), "engine": np.array(data.engine),
              "temperature_K": np.array(math.nan if data.temperature_K is None else data.temperature_K),
              "nhc_eta": nhc.get("eta", np.zeros(0)), "nhc_p_eta": nhc.get("p_eta", np.zeros(0))}
    record.update({name: getattr(data, name) for name in _ARRAY_FIELDS})
    record.update({name: np.array(json.dumps(getattr(data, name))) for name in _JSON_FIELDS})
    return record


def _decode_restart(files) -> RestartData:
    if str(files["format"]) != RESTART_FORMAT:
        raise ValueError(f"not a {RESTART_FORMAT} restart file")
    values = {name: files[name] for name in _ARRAY_FIELDS}
    values.update({name: json.loads(str(files[name])) for name in _JSON_FIELDS})
    target = float(files["temperature_K"])
    values.update(energy=files["potential_energy"], step=int(files["step"]),
                  temperature_K=None if math.isnan(target) else target,
                  engine=str(files["engine"]) if "engine" in files.files else "domain")
    values["nhc_state"] = None
    if values["parameters"]["ensemble"] == "nvt_nhc":
        values["nhc_state"] = {"temperature_K": target, "eta": np.array(files["nhc_eta"]),
                               "p_eta": np.array(files["nhc_p_eta"])}
    return RestartData(**{f.name: values[f.name] for f in fields(RestartData)})


def read_restart(path) -> RestartData:
    """Parse a restart file (format tag checked; a file without ``engine`` reads as "domain")."""
    with np.load(path) as files:
        return _decode_restart(files)


def write_restart(path, data: RestartData) -> None:
    """Write ``data`` as an ``.npz``, atomically: a sibling temporary file, then a rename."""
    path = Path(path)
    scratch = path.with_name(path.name + ".tmp.npz")
    np.savez(scratch, **_encode_restart(data))
    os.replace(scratch, path)


def resume_mismatch(saved: dict, requested: dict, *, ignore=()) -> dict:
    """``{key: (saved, requested)}`` for every parameter a continuation changes, in sorted key
    order; ``total_steps`` and the keys in ``ignore`` are not compared."""
    skipped = {"total_steps", *ignore}
    keys = sorted((saved.keys() | requested.keys()) - skipped)
    return {k: (saved.get(k), requested.get(k)) for k in keys if saved.get(k) != requested.get(k)}


# ------------------------------------------------------------------------------------ outputs
@dataclass(frozen=True)
class Every:
    """An output period: ``period`` 0 disables it; ``and_last`` also fires at the run's final step."""

    period: int
    and_last: bool

    def fires(self, step: int, last_step: int | None) -> bool:
        if self.period <= 0:
            return False
        return step % self.period == 0 or (self.and_last and last_step is not None and step == last_step)


class MDOutputs:
    """A driver's output files: a thermo row every ``thermo_interval`` steps, an EXTXYZ frame every
    ``xyz_interval``, the restart file every ``restart_interval`` (0 disables each; no
    ``output_dir`` disables all); the final step (``total_steps``) always gets a thermo row and a
    restart. A fresh start clears earlier outputs and writes the step-0 frame and restart; a resume
    passes the restart's ``offsets`` and the tracked files are cut back to them.

    ``source`` (the driver) provides ``nsteps``, ``parameters``, ``cell``, ``device``,
    ``md_fields()``, ``thermodynamics()`` and ``thermostat_state()``."""

    TRACKED = (THERMO_FILE, TRAJECTORY_FILE)

    def __init__(self, source, output_dir, thermo_interval: int, xyz_interval: int, restart_interval: int,
                 total_steps: int | None, offsets: dict | None, *, engine: str = "native"):
        self.source = weakref.proxy(source)
        self.engine = engine
        self.total_steps = total_steps
        self.thermo_interval, self.xyz_interval, self.restart_interval = (
            int(thermo_interval), int(xyz_interval), int(restart_interval))
        self.schedule = {"thermo": Every(self.thermo_interval, True), "frame": Every(self.xyz_interval, False),
                         "restart": Every(self.restart_interval, True)}
        self.output_dir = None if output_dir is None else Path(output_dir)
        self.logger = None
        self.files: dict[str, Path] = {}
        if self.output_dir is None:
            return
        self.output_dir.mkdir(parents=True, exist_ok=True)
        self.files = {name: self.output_dir / name for name in self.TRACKED}
        if offsets is None:
            self._start_fresh()
        else:
            self._cut_back(offsets)
        if self.xyz_interval:
            self.logger = self._open_frame_logger(append=offsets is not None)
        if offsets is None:
            self._emit({kind for kind in ("frame", "restart") if self.schedule[kind].period}, None)

    # ---------------------------------------------------------------- set-up
    def _start_fresh(self) -> None:
        for path in (*self.files.values(), self.output_dir / RESTART_FILE):
            path.unlink(missing_ok=True)
        self.files[THERMO_FILE].write_text(THERMO_HEADER)

    def _cut_back(self, offsets: dict) -> None:
        """Truncate each tracked file that exists to the size the restart recorded."""
        present = {name: path for name, path in self.files.items() if name in offsets and path.exists()}
        too_short = sorted(name for name, path in present.items() if path.stat().st_size < int(offsets[name]))
        if too_short:
            raise ValueError(f"cannot resume: {', '.join(too_short)} ended before the restart file's recorded "
                             "size (the outputs are older than the restart)")
        for name, path in present.items():
            os.truncate(path, int(offsets[name]))

    def _open_frame_logger(self, append: bool):
        from fastmd_amd.execution.gpu_logging import AsyncGPUMDLogger, AtomsTemplate

        fields_ = self.source.md_fields()
        template = AtomsTemplate(numbers=fields_["numbers"].cpu().numpy(),
                                 masses=fields_["masses"].double().cpu().numpy(),
                                 cell=self.source.cell.detach().cpu().double().numpy(), pbc=np.ones(3, bool),
                                 explicit_masses=bool(getattr(self.source, "explicit_masses", False)))
        tchain = int(self.source.parameters["tchain"])
        extras = {"step": 1, "time_fs": 1, "target_temp_K": 1, "nhc_eta": tchain, "nhc_p_eta": tchain,
                  "nhc_conserved_energy": 1}
        trajectory = ExtxyzTrajectory(self.files[TRAJECTORY_FILE], append=append)
        try:
            return AsyncGPUMDLogger(template, self.source.device, trajectory=trajectory,
                                    state_dtype=fields_["positions"].dtype, extras=extras)
        except BaseException:
            trajectory.close()
            raise

    # ---------------------------------------------------------------- per step
    def due_kinds(self, step: int) -> set:
        """The output kinds ("thermo", "frame", "restart") due at ``step``."""
        if self.output_dir is None:
            return set()
        return {kind for kind, every in self.schedule.items() if every.fires(step, self.total_steps)}

    def due(self, step: int) -> bool:
        """Whether the step writes any output (the driver settles such windows on their own)."""
        return bool(self.due_kinds(step))

    def write(self) -> dict | None:
        """The outputs due at the current step (call after every step); returns the thermodynamics
        they used, or None when nothing was due."""
        kinds = self.due_kinds(self.source.nsteps)
        if not kinds:
            return None
        thermo = self.source.thermodynamics()
        self._emit(kinds, thermo)
        return thermo

    def _emit(self, kinds: set, thermo: dict | None) -> None:
        if "thermo" in kinds:
            with open(self.files[THERMO_FILE], "a") as stream:
                stream.write(thermo_row(self.source.nsteps, thermo))
        if "frame" in kinds:
            self.log_frame(thermo)
        if "restart" in kinds:
            self.save_restart(None)

    def log_frame(self, thermo: dict | None = None) -> None:
        """Queue the current frame on the EXTXYZ logger (the file write is asynchronous)."""
        if self.logger is None:
            raise RuntimeError("log_frame needs an output_dir and a nonzero xyz_interval")
        thermo = self.source.thermodynamics() if thermo is None else thermo
        state = self.source.md_fields()
        as64 = lambda *values: torch.tensor(values, dtype=torch.float64)  # noqa: E731
        extras = {"step": as64(thermo["step"]), "time_fs": as64(thermo["time_fs"]),
                  "target_temp_K": as64(thermo["target_temperature"]), "nhc_eta": as64(*thermo["eta"]),
                  "nhc_p_eta": as64(*thermo["p_eta"]), "nhc_conserved_energy": as64(thermo["conserved_energy"])}
        self.logger.enqueue(step=thermo["step"], time_ps=thermo["time_fs"] / 1000.0, positions=state["positions"],
                            momenta=state["momenta"], forces=state["forces"], cell=self.source.cell,
                            potential_energy=as64(thermo["potential_energy"]),
                            kinetic_energy=as64(thermo["kinetic_energy"]), temperature=as64(thermo["temperature"]),
                            extras=extras)

    def save_restart(self, path=None) -> None:
        """Write the current state, the thermostat and the tracked files' sizes (after the queued
        frames are on disk) to the restart file (default: in ``output_dir``)."""
        if path is None:
            if self.output_dir is None:
                raise ValueError("save_restart needs a path when there is no output_dir")
            path = self.output_dir / RESTART_FILE
        if self.logger is not None:
            self.logger.flush()
        state = self.source.md_fields()
        thermostat = self.source.thermostat_state()
        host = {key: value.detach().cpu() for key, value in state.items()}
        write_restart(path, RestartData(
            ids=host["ids"].long().numpy(), numbers=host["numbers"].long().numpy(),
            masses=host["masses"].double().numpy(), positions=host["positions"].double().numpy(),
            momenta=host["momenta"].double().numpy(), forces=host["forces"].numpy(), energy=host["energy"].numpy(),
            reference_energy=host["reference_energy"].numpy(), cell=self.source.cell.detach().cpu().numpy(),
            pbc=np.ones(3, dtype=bool), step=self.source.nsteps, parameters=self.source.parameters,
            temperature_K=thermostat.get("temperature_K"), nhc_state=thermostat,
            offsets={name: p.stat().st_size if p.exists() else 0 for name, p in self.files.items()},
            engine=self.engine))

    def close(self) -> None:
        logger, self.logger = self.logger, None
        if logger is not None:
            logger.close()

    def close_quietly(self) -> None:
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass
