"""The reference's multi-system entry point (fastmd/interfaces/multi_system_md.py:78-125,
``MultiSystemMolecularDynamics``) on the slot union of ``fastmd_amd.execution.system_batch``.

Same argument names and meanings for the NVT Nose-Hoover chain ensemble: ``model`` first, then the
systems; ``momenta`` one (n_s, 3) array per system, default Maxwell-Boltzmann at ``temperature``
with ``seed + s``; ``slot_atoms`` the slots' atom ceilings (None, one int for every slot, or one per
system); ``tdamp`` defaults to ``taut``. All systems run as one union, so ``union_rows`` is only
checked against it. Other ensembles, adapter loading by name and the trajectory/log files of the
reference's union driver raise ``NotImplementedError``.
"""
from __future__ import annotations

import numpy as np

from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
from fastmd_amd.execution.system_batch import SystemBatchedMD, _system_arrays


def _ceilings(slot_atoms, counts) -> tuple:
    if slot_atoms is None:
        return tuple(counts)
    if isinstance(slot_atoms, (int, np.integer)):
        return tuple(max(int(slot_atoms), n) for n in counts)
    ceilings = tuple(int(c) for c in slot_atoms)
    if len(ceilings) != len(counts) or any(c < n for c, n in zip(ceilings, counts)):
        raise ValueError("slot_atoms: one ceiling per system, at least its atom count")
    return ceilings


class MultiSystemMolecularDynamics(SystemBatchedMD):
    """S different systems advanced together in slots of one whole-step graph."""

    def __init__(self, model, systems, *, momenta=None, ensemble: str = "nvt_nhc", temperature: float = 300.0,
                 timestep: float = 1.0, taut: float = 100.0, tdamp: float | None = None, tchain: int = 3,
                 tloop: int = 1, fix_com: bool | None = None, seed: int = 0, steps_per_launch: int = 10,
                 slot_atoms=None, union_rows: int | None = None, capacity_headroom: float | None = None,
                 config=None, model_path: str | None = None, model_dtype: str | None = None, device=None,
                 trajectory=None, logfile=None, loginterval: int | None = None, **unsupported) -> None:
        if ensemble != "nvt_nhc":
            raise NotImplementedError(f"ensemble {ensemble!r}: this build integrates the Nose-Hoover chain only")
        if isinstance(model, str) or model_path is not None or model_dtype not in (None, "float32"):
            raise NotImplementedError("adapters are passed as objects (no loading by name or path)")
        if fix_com or trajectory is not None or logfile is not None or loginterval is not None or unsupported:
            raise NotImplementedError("centre-of-mass fixing and the union driver's trajectory/log files are "
                                      "not supported")
        systems = list(systems)
        counts = [int(_system_arrays(a)[0].shape[0]) for a in systems]
        ceilings = _ceilings(slot_atoms, counts)
        if union_rows is not None and sum(ceilings) > int(union_rows):
            raise NotImplementedError(f"{sum(ceilings)} rows in one union exceed union_rows={union_rows}: "
                                      "several unions are not supported")
        if momenta is None:
            momenta = [maxwell_boltzmann_momenta(_system_arrays(a)[3], temperature, seed + s)
                       for s, a in enumerate(systems)]
        super().__init__(systems, model, ceilings=ceilings, device="cuda" if device is None else device,
                         temperature=temperature, timestep=timestep, tdamp=taut if tdamp is None else tdamp,
                         tchain=tchain, tloop=tloop, momenta=momenta, steps_per_launch=steps_per_launch,
                         config=config)
