"""(e) ASE ``NoseHooverChainNVT`` on the GPU: fused HIP velocity-Verlet + NHC half steps.

Interface of the reference's ``GPUNoseHooverChainNVT`` (fastmd/execution/gpu_nhc.py:709-1407)
for the single-device protocol: the float64 state lives in ONE flat device buffer
``[q 3N | p 3N | F 3N | eta tchain | p_eta tchain | E 1]`` (NHCState, :216-267) so a
transactional backup/restore is one copy; a step is ``step_pre_force`` (NHC(dt/2), kick with
the cached F(q_n), drift) then ``step_post_force(F, E)`` (kick, NHC(dt/2), cache F), each ONE
kernel launch (``fmd_nhc_pre_force`` / ``fmd_nhc_post_force``) up to 4096 atoms and three
grid-wide kernels beyond (the reference's fused kernels are single-CTA and limited to
3N <= 16 384, :96,839-849, beyond which it runs several hundred torch ops per step). Constants: ``nhc_constants`` forms ASE's scalars
with ASE's own Python expressions (:113-133) and ``set_temperature`` rewrites them on the device
without a host sync. ``backend="torch"`` is not offered: the CPU restatement of the algorithm is
the test oracle (oracle/nhc.py), not a product path.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from fastmd_amd import _abi, units
from fastmd_amd.execution.gpu_integrator import StatefulIntegrator, _PinnedUpload
from fastmd_amd._roctx import roctx_ranged

FOURTH_ORDER_COEFFS = [
    1 / (2 - 2 ** (1 / 3)),
    -(2 ** (1 / 3)) / (2 - 2 ** (1 / 3)),
    1 / (2 - 2 ** (1 / 3)),
]
_C_Q = 16
_MAX_CHAIN = 8


@dataclass(frozen=True)
class NHCConstants:
    kT: float
    ndof_kT: float
    Q: np.ndarray
    dt2: float
    sub: list
    values: list


def nhc_constants(n_atoms: int, *, temperature_K: float, timestep: float, tdamp: float, tchain: int,
                  tloop: int) -> NHCConstants:
    """ASE's thermostat scalars with ASE's expressions (gpu_nhc.py:113-133); ``values`` is the
    device layout [dt, dt/2, kT, 3NkT, 3 x (delta, delta/2, -(delta/4), -delta), Q, 1/Q]."""
    n = int(n_atoms)
    kT = units.kB * temperature_K
    Q = np.zeros(tchain)
    Q[0] = 3 * n * kT * tdamp ** 2
    Q[1:] = kT * tdamp ** 2
    ndof_kT = 3 * n * kT
    dt2 = timestep / 2
    sub = []
    for coeff in FOURTH_ORDER_COEFFS:
        delta = coeff * dt2 / tloop
        sub.append((delta, delta / 2, -(delta / 4), -delta))
    values = [timestep, dt2, kT, ndof_kT]
    for entry in sub:
        values.extend(entry)
    values.extend(Q.tolist())
    values.extend((1.0 / Q).tolist())
    return NHCConstants(kT, ndof_kT, Q, dt2, sub, values)


def maxwell_boltzmann_momenta(masses, temperature_K: float, seed=0) -> np.ndarray:
    """ASE ``MaxwellBoltzmannDistribution(atoms, temperature_K=T, rng=default_rng(seed))`` momenta,
    bit for bit (gpu_nhc.py:199-213): p = xi * sqrt(m kB T), xi standard normal (N, 3)."""
    masses = np.asarray(masses, dtype=np.float64).reshape(-1)
    rng = seed if isinstance(seed, np.random.Generator) else np.random.default_rng(seed)
    temp = units.kB * temperature_K
    xi = rng.standard_normal((len(masses), 3))
    return xi * np.sqrt(masses * temp)[:, np.newaxis]


@dataclass
class NHCState:
    """Views into one flat float64 buffer (gpu_nhc.py:216-267)."""

    flat: Tensor
    positions: Tensor
    momenta: Tensor
    forces: Tensor
    eta: Tensor
    p_eta: Tensor
    potential_energy: Tensor

    @staticmethod
    def allocate(n_atoms: int, tchain: int, device) -> "NHCState":
        n3 = 3 * n_atoms
        flat = torch.zeros(3 * n3 + 2 * tchain + 1, dtype=torch.float64, device=device)
        o = 0
        positions = flat[o:o + n3].view(n_atoms, 3)
        o += n3
        momenta = flat[o:o + n3].view(n_atoms, 3)
        o += n3
        forces = flat[o:o + n3].view(n_atoms, 3)
        o += n3
        eta = flat[o:o + tchain]
        o += tchain
        p_eta = flat[o:o + tchain]
        o += tchain
        energy = flat[o:o + 1]
        return NHCState(flat, positions, momenta, forces, eta, p_eta, energy)

    def numpy(self) -> dict:
        return {
            "positions": self.positions.detach().cpu().numpy().copy(),
            "momenta": self.momenta.detach().cpu().numpy().copy(),
            "forces": self.forces.detach().cpu().numpy().copy(),
            "eta": self.eta.detach().cpu().numpy().copy(),
            "p_eta": self.p_eta.detach().cpu().numpy().copy(),
            "potential_energy": float(self.potential_energy.item()),
        }


class GPUNoseHooverChainNVT(StatefulIntegrator):
    """ASE-exact NHC NVT on one MI355X (see the module docstring). Parameters mirror ASE:
    ``timestep``/``tdamp`` in ASE time units (e.g. ``0.25 * units.fs``), ``temperature_K``,
    ``tchain``, ``tloop``; ``masses`` (N,) amu; ``positions``/``momenta`` (N, 3) float64.
    ``force_dtype=torch.float32`` with ``numpy_kick_semantics`` forms the kick dt/2*F in float32
    like NumPy 2 (NEP 50) does for float32 forces (gpu_nhc.py:380-384)."""

    ensemble = "nvt_nhc"

    def __init__(self, masses, positions, momenta, *, temperature_K: float, timestep: float, tdamp: float,
                 tchain: int = 3, tloop: int = 1, forces=None, potential_energy=None, device="cuda",
                 backend: str = "auto", force_dtype: torch.dtype = torch.float64, numpy_kick_semantics: bool = True,
                 fast_math: bool = False, comm=None, n_global: int | None = None, capacity: int | None = None,
                 protocol: str = "auto", fix_com: bool = False) -> None:
        if tchain < 1 or tloop < 1:
            raise ValueError("tchain and tloop must be >= 1")
        if tchain > _MAX_CHAIN:
            raise ValueError(f"tchain must be <= {_MAX_CHAIN}")
        if tdamp <= 0 or timestep < 0:
            raise ValueError("tdamp must be positive and timestep non-negative")
        if protocol not in ("auto", "single") or comm is not None or fix_com:
            raise NotImplementedError("the decomposed (P>1) protocol is not part of the one-GPU build")
        if backend not in ("auto", "hip"):
            raise ValueError(f"unknown backend {backend!r} (the fused HIP kernels are the only backend)")
        if fast_math:
            raise NotImplementedError("fast_math is not offered: the kernels are ASE-exact")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("GPUNoseHooverChainNVT runs on the GPU")
        _abi.load()
        masses_np = np.asarray(masses.detach().cpu().numpy() if torch.is_tensor(masses) else masses,
                               dtype=np.float64).reshape(-1)
        self.n_atoms = n = int(masses_np.shape[0])
        if n_global not in (None, n) or capacity not in (None, n):
            raise NotImplementedError("n_global/capacity belong to the decomposed protocol")
        self.tchain = int(tchain)
        self.tloop = int(tloop)
        self.temperature_K = float(temperature_K)
        self.dt = float(timestep)
        self.tdamp = float(tdamp)
        self.force_dtype = force_dtype
        self.f32_kick = bool(numpy_kick_semantics and force_dtype == torch.float32)
        self.backend = "hip"
        self.protocol = "single"
        self.comm = None
        self._init_constants(n)
        self.masses = torch.tensor(masses_np, dtype=torch.float64, device=self.device).reshape(n, 1).contiguous()
        self.state = NHCState.allocate(n, self.tchain, self.device)
        self._backup = NHCState.allocate(n, self.tchain, self.device)
        self._work = torch.zeros(int(_abi.load().fmd_nhc_work_size(n)), dtype=torch.float64, device=self.device)
        self.set_state(positions=positions, momenta=momenta, forces=forces, potential_energy=potential_energy)

    # -------------------------------------------------------------- constants
    def _constants(self, temperature_K: float) -> NHCConstants:
        return nhc_constants(self.n_atoms, temperature_K=temperature_K, timestep=self.dt, tdamp=self.tdamp,
                             tchain=self.tchain, tloop=self.tloop)

    def _init_constants(self, n: int) -> None:
        c = self._constants(self.temperature_K)
        self._keep(c, self.temperature_K)
        self.consts = torch.tensor(c.values, dtype=torch.float64, device=self.device)
        self.Q = self.consts[_C_Q:_C_Q + self.tchain]
        self._upload = _PinnedUpload(self.consts)

    def _keep(self, c: NHCConstants, temperature_K: float) -> None:
        self.temperature_K = temperature_K
        self.kT, self.ndof_kT, self.Q_np, self.dt2, self.sub = c.kT, c.ndof_kT, c.Q, c.dt2, c.sub

    def set_temperature(self, temperature_K: float) -> None:
        """New target temperature: the constructor's expressions, uploaded without a host sync;
        ``set_temperature(T)`` equals a fresh integrator at T bitwise (gpu_nhc.py:156-167)."""
        temperature_K = float(temperature_K)
        c = self._constants(temperature_K)
        self._upload(c.values)
        self._keep(c, temperature_K)

    def target_row(self, temperature_K: float) -> list[float]:
        return list(self._constants(float(temperature_K)).values)

    def load_target_row(self, row: Tensor) -> None:
        self.consts.copy_(row)

    def state_dict(self) -> dict:
        return {"eta": self.eta.detach().cpu().numpy().copy(), "p_eta": self.p_eta.detach().cpu().numpy().copy(),
                "temperature_K": self.temperature_K}

    @torch.no_grad()
    def load_state_dict(self, state: dict) -> None:
        eta = torch.as_tensor(np.asarray(state["eta"], dtype=np.float64))
        p_eta = torch.as_tensor(np.asarray(state["p_eta"], dtype=np.float64))
        if eta.shape != (self.tchain,) or p_eta.shape != (self.tchain,):
            raise ValueError(f"eta/p_eta must have shape ({self.tchain},)")
        self.set_temperature(float(state["temperature_K"]))
        self.eta.copy_(eta)
        self.p_eta.copy_(p_eta)

    # -------------------------------------------------------------- state
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

    def _as_f64(self, x) -> Tensor:
        if torch.is_tensor(x):
            return x.detach().to(device=self.device, dtype=torch.float64)
        return torch.as_tensor(np.asarray(x, dtype=np.float64), device=self.device)

    @torch.no_grad()
    def set_state(self, *, positions=None, momenta=None, forces=None, eta=None, p_eta=None, potential_energy=None,
                  state: NHCState | None = None) -> None:
        st = self.state if state is None else state
        n = self.n_atoms
        if positions is not None:
            st.positions.copy_(self._as_f64(positions).reshape(n, 3))
        if momenta is not None:
            st.momenta.copy_(self._as_f64(momenta).reshape(n, 3))
        if forces is not None:
            st.forces.copy_(self._as_f64(forces).reshape(n, 3))
        if eta is not None:
            st.eta.copy_(self._as_f64(eta).reshape(-1))
        if p_eta is not None:
            st.p_eta.copy_(self._as_f64(p_eta).reshape(-1))
        if potential_energy is not None:
            st.potential_energy.copy_(self._as_f64(potential_energy).reshape(1))

    @torch.no_grad()
    def set_forces(self, forces, energy=None, state: NHCState | None = None) -> None:
        st = self.state if state is None else state
        n = self.n_atoms
        st.forces.copy_(forces.reshape(n, 3) if torch.is_tensor(forces) else self._as_f64(forces).reshape(n, 3))
        if energy is not None:
            st.potential_energy.copy_(energy.reshape(1) if torch.is_tensor(energy)
                                      else self._as_f64(energy).reshape(1))

    # -------------------------------------------------------------- step halves
    @roctx_ranged("gpu_integrator")
    def step_pre_force(self, state: NHCState | None = None) -> Tensor:
        """NHC(dt/2); p += dt/2 * F(q_n); q += dt * p / m. Returns the float64 positions view."""
        st = self.state if state is None else state
        _abi.call("fmd_nhc_pre_force", st.positions.data_ptr(), st.momenta.data_ptr(), st.forces.data_ptr(),
                  self.masses.data_ptr(), st.eta.data_ptr(), st.p_eta.data_ptr(), self.consts.data_ptr(),
                  self.n_atoms, self.tchain, self.tloop, 1 if self.f32_kick else 0, self._work.data_ptr(),
                  _abi.stream_handle(self.device))
        return st.positions

    def _post_inputs(self, forces: Tensor, energy: Tensor | None):
        """Forces as a contiguous float32/float64 [N, 3] on this device and the energy's kind."""
        forces = forces.reshape(self.n_atoms, 3)
        if forces.dtype not in (torch.float32, torch.float64):
            forces = forces.to(torch.float32)
        if not forces.is_contiguous():
            forces = forces.contiguous()
        if forces.device != self.device:
            raise ValueError("forces must be on the integrator's device")
        e_kind = 0
        if energy is not None:
            energy = energy.reshape(-1)
            if energy.dtype not in (torch.float32, torch.float64):
                energy = energy.to(torch.float64)
            e_kind = 2 if energy.dtype == torch.float64 else 1
        return forces, 1 if forces.dtype == torch.float64 else 0, energy, e_kind

    @roctx_ranged("gpu_integrator")
    def step_post_force(self, forces: Tensor, energy: Tensor | None = None, state: NHCState | None = None) -> None:
        """p += dt/2 * F(q_{n+1}); NHC(dt/2); cache F (float64) and the energy."""
        st = self.state if state is None else state
        forces, f64, energy, e_kind = self._post_inputs(forces, energy)
        _abi.call("fmd_nhc_post_force", st.momenta.data_ptr(), forces.data_ptr(), f64, st.forces.data_ptr(),
                  self.masses.data_ptr(),
                  st.eta.data_ptr(), st.p_eta.data_ptr(), self.consts.data_ptr(), _abi.ptr(energy), e_kind,
                  st.potential_energy.data_ptr(), self.n_atoms, self.tchain, self.tloop,
                  1 if self.f32_kick else 0, self._work.data_ptr(), _abi.stream_handle(self.device))

    @roctx_ranged("gpu_integrator")
    def step_post_pre(self, forces: Tensor, energy: Tensor | None = None, state: NHCState | None = None) -> Tensor:
        """``step_post_force(forces, energy)`` then the next step's ``step_pre_force()`` in one launch
        (fmd_nhc_post_pre; the same state bit for bit). Returns the float64 positions view."""
        st = self.state if state is None else state
        forces, f64, energy, e_kind = self._post_inputs(forces, energy)
        _abi.call("fmd_nhc_post_pre", st.positions.data_ptr(), st.momenta.data_ptr(), forces.data_ptr(), f64,
                  st.forces.data_ptr(), self.masses.data_ptr(), st.eta.data_ptr(), st.p_eta.data_ptr(),
                  self.consts.data_ptr(), _abi.ptr(energy), e_kind, st.potential_energy.data_ptr(), self.n_atoms,
                  self.tchain, self.tloop, 1 if self.f32_kick else 0, self._work.data_ptr(),
                  _abi.stream_handle(self.device))
        return st.positions

    def step(self, force_fn, state: NHCState | None = None):
        st = self.state if state is None else state
        q = self.step_pre_force(st)
        result = force_fn(q)
        forces, energy = result if isinstance(result, tuple) else (result, None)
        self.step_post_force(forces, energy=energy, state=st)
        return st.positions, st.momenta, st.forces

    # -------------------------------------------------------------- observables (logging only)
    def velocities(self, state: NHCState | None = None) -> Tensor:
        st = self.state if state is None else state
        return st.momenta / self.masses

    def kinetic_energy(self, state: NHCState | None = None) -> Tensor:
        """0.5 * vdot(p, p/m) (``Atoms.get_kinetic_energy``), 0-dim float64."""
        st = self.state if state is None else state
        return 0.5 * (st.momenta * (st.momenta / self.masses)).sum()

    def temperature(self, state: NHCState | None = None) -> Tensor:
        return 2 * self.kinetic_energy(state) / (3 * self.n_atoms * units.kB)

    def thermostat_energy(self, state: NHCState | None = None, constants: tuple | None = None) -> Tensor:
        """``NoseHooverChainThermostat.get_thermostat_energy`` (gpu_nhc.py:1224-1231)."""
        st = self.state if state is None else state
        kT, ndof_kT, Q = (self.kT, self.ndof_kT, self.Q) if constants is None else constants
        return ndof_kT * st.eta[0] + kT * st.eta[1:].sum() + (0.5 * (st.p_eta * st.p_eta) / Q).sum()

    def conserved_energy(self, potential_energy=None, state: NHCState | None = None,
                         constants: tuple | None = None) -> Tensor:
        """E_pot + E_kin + E_thermostat (ASE ``get_conserved_energy``)."""
        st = self.state if state is None else state
        epot = st.potential_energy[0] if potential_energy is None else potential_energy
        return epot + self.kinetic_energy(st) + self.thermostat_energy(st, constants=constants)

    # -------------------------------------------------------------- transactions
    def backup(self, state: NHCState | None = None) -> None:
        self._backup.flat.copy_((self.state if state is None else state).flat)

    def restore(self, state: NHCState | None = None) -> None:
        (self.state if state is None else state).flat.copy_(self._backup.flat)

    def snapshot(self) -> tuple:
        return self.state.flat.clone(), self._backup.flat.clone()

    def load_snapshot(self, snapshot: tuple) -> None:
        state, backup = snapshot
        self.state.flat.copy_(state)
        self._backup.flat.copy_(backup)

    def new_state(self) -> NHCState:
        return NHCState.allocate(self.n_atoms, self.tchain, self.device)

    def positions32(self) -> Tensor:
        return self.state.positions.to(torch.float32)

    def warmup_compile(self, force_dtypes=None, energy_dtype=torch.float32) -> None:
        """No JIT here (the kernels are compiled ahead of time); kept for interface parity."""
        return None
