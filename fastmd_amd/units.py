"""ASE units (CODATA 2014, ASE's default), computed from the constants: eV, Å, amu, K.

The reference takes ``ase.units`` (fastmd/execution/gpu_nhc.py:70); ASE is not a dependency
here, so the two constants the MD step uses are formed with ASE's own expressions.
"""
from __future__ import annotations

import math

_e = 1.6021766208e-19  # C (elementary charge)
_amu = 1.660539040e-27  # kg
_k = 1.38064852e-23  # J/K (Boltzmann)

kB = _k / _e  # eV/K
second = 1e10 * math.sqrt(_e / _amu)  # ASE time unit per second
fs = 1e-15 * second
