"""Nose-Hoover chain oracle (test infrastructure only; see oracle/__init__.py).

A NumPy float64 restatement of ASE 3.29 ``NoseHooverChainNVT.step`` in the reference's op order
(the torch backend fastmd/execution/gpu_nhc.py:1165-1195, the Triton kernels :315-425): per half
step, ``integrate_nhc``: ke2 = sum(p**2 / m); for each Suzuki-Yoshida coefficient: p_eta_j
sweeps j = M-1..0, eta += delta * p_eta / Q, p *= exp(-delta * p_eta0 / Q0), ke2 recomputed,
p_eta_j sweeps j = 0..M-1. Constants from ``fastmd_amd.execution.gpu_nhc.nhc_constants``-equal
expressions (restated here so the oracle does not import the product).
"""
from __future__ import annotations

import numpy as np

KB = 1.38064852e-23 / 1.6021766208e-19
FS = 1e-15 * 1e10 * np.sqrt(1.6021766208e-19 / 1.660539040e-27)
FOURTH_ORDER_COEFFS = [1 / (2 - 2 ** (1 / 3)), -(2 ** (1 / 3)) / (2 - 2 ** (1 / 3)), 1 / (2 - 2 ** (1 / 3))]


def constants(n_atoms, temperature_K, timestep, tdamp, tchain, tloop):
    kT = KB * temperature_K
    Q = np.zeros(tchain)
    Q[0] = 3 * n_atoms * kT * tdamp ** 2
    Q[1:] = kT * tdamp ** 2
    sub = []
    for coeff in FOURTH_ORDER_COEFFS:
        delta = coeff * (timestep / 2) / tloop
        sub.append((delta, delta / 2, -(delta / 4), -delta))
    return kT, 3 * n_atoms * kT, Q, sub


class NHC:
    """State: q, p (N,3) float64, F (cached, float64), eta, p_eta (tchain,), E."""

    def __init__(self, masses, q, p, *, temperature_K, timestep, tdamp, tchain=3, tloop=1, f32_kick=False,
                 forces=None, energy=0.0):
        self.m = np.asarray(masses, dtype=np.float64).reshape(-1, 1)
        self.q = np.array(q, dtype=np.float64)
        self.p = np.array(p, dtype=np.float64)
        self.f = np.zeros_like(self.q) if forces is None else np.array(forces, dtype=np.float64)
        self.e = float(energy)
        self.dt = float(timestep)
        self.tchain, self.tloop = int(tchain), int(tloop)
        self.f32_kick = bool(f32_kick)
        self.eta = np.zeros(tchain)
        self.p_eta = np.zeros(tchain)
        self.set_temperature(temperature_K, tdamp)

    def set_temperature(self, temperature_K, tdamp=None):
        self.tdamp = self.tdamp if tdamp is None else float(tdamp)
        self.kT, self.ndof_kT, self.Q, self.sub = constants(self.q.shape[0], float(temperature_K), self.dt,
                                                            self.tdamp, self.tchain, self.tloop)

    def _ke2(self):
        return np.sum(self.p * self.p / self.m)

    def _p_eta_j(self, j, ke2, delta2, neg_delta4):
        pe, Q, M = self.p_eta, self.Q, self.tchain
        if j < M - 1:
            s = np.exp(pe[j + 1] * neg_delta4 / Q[j + 1])
            pe[j] *= s
        g = ke2 - self.ndof_kT if j == 0 else pe[j - 1] * pe[j - 1] / Q[j - 1] - self.kT
        pe[j] += g * delta2
        if j < M - 1:
            pe[j] *= s

    def integrate_nhc(self):
        M = self.tchain
        ke2 = self._ke2()
        for _ in range(self.tloop):
            for delta, delta2, neg_delta4, neg_delta in self.sub:
                for j in range(M):
                    self._p_eta_j(M - j - 1, ke2, delta2, neg_delta4)
                self.eta += self.p_eta * delta / self.Q
                self.p *= np.exp(self.p_eta[0] * neg_delta / self.Q[0])
                ke2 = self._ke2()
                for j in range(M):
                    self._p_eta_j(j, ke2, delta2, neg_delta4)

    def _kick(self, forces):
        if self.f32_kick:
            self.p += (np.float32(self.dt / 2) * np.asarray(forces, dtype=np.float32)).astype(np.float64)
        else:
            self.p += np.asarray(forces, dtype=np.float64) * (self.dt / 2)

    def pre_force(self):
        self.integrate_nhc()
        self._kick(self.f)
        self.q += self.p * self.dt / self.m
        return self.q

    def post_force(self, forces, energy=None):
        self._kick(forces)
        self.integrate_nhc()
        self.f = np.asarray(forces, dtype=np.float64).copy()
        if energy is not None:
            self.e = float(energy)

    def step(self, force_fn):
        q = self.pre_force()
        forces, energy = force_fn(q)
        self.post_force(forces, energy)

    def kinetic_energy(self):
        return 0.5 * np.sum(self.p * (self.p / self.m))

    def thermostat_energy(self):
        return (self.ndof_kT * self.eta[0] + self.kT * self.eta[1:].sum()
                + np.sum(0.5 * self.p_eta * self.p_eta / self.Q))

    def conserved_energy(self):
        return self.e + self.kinetic_energy() + self.thermostat_energy()


def harmonic(q0, k, dtype=np.float64):
    """Springs to q0 (tests/test_gpu_nhc.py:99-118): forces -k (q - q0), energy k/2 |q - q0|^2."""
    q0 = np.asarray(q0)

    def fn(q):
        if dtype == np.float32:
            d = q.astype(np.float32) - q0.astype(np.float32)
            f = np.float32(-k) * d
        else:
            d = q - q0
            f = -k * d
        return f, 0.5 * k * float(np.sum(d.astype(np.float64) ** 2))

    return fn
