"""CPU oracle of the three-body Fourier angle basis (test infrastructure only: imported by tests,
``__graft_entry__.smoke()`` and the bench's CPU baseline, never by the product path).

Restates ``fastmd/models/matris/op/triton_threebody_fourier.py``:

- forward (:1-10 docstring, :47-88 kernel, :273-298 torch path): for row t with bond vectors
  a = u[target[t]], b = u[source[t]],
  ``c = (a . b) (1 - 1e-6)``, ``theta = acos(c)``,
  ``out[t] = [1/sqrt(2), sin(theta f_1..F), cos(theta f_1..F)] / scale``; the model's
  ``FourierExpansion`` (basis_function.py:102-136) sets f = 1..max_f and scale = sqrt(pi);
- VJP (:99-166 kernel, :169-181 ordered torch form): ``dtheta = sum_k (g_sin_k cos(theta f_k)
  - g_cos_k sin(theta f_k)) f_k / scale``, ``d = -dtheta / sqrt(max(1 - c^2, 1e-24)) (1 - 1e-6)``,
  ``g_u[target[t]] += d b``, ``g_u[source[t]] += d a``.

Pinned in tests/test_threebody.py by what the mathematics fixes, not by restating these lines:
closed-form angles (orthogonal, 60 degrees, parallel and antiparallel vectors), invariance of
the basis under a common rotation, the VJP against central finite differences and against
torch's autograd of an independent float64 composition, and the VJP's bilinearity in (g, u).
"""
from __future__ import annotations

import numpy as np

EPS_SCALE = 1.0 - 1.0e-6


def fourier_basis(u, target, source, freqs, scale, dtype=np.float64) -> np.ndarray:
    """out [rows, 1 + 2F] in ``dtype`` arithmetic (float64 by default)."""
    u = np.asarray(u, dtype)
    freqs = np.asarray(freqs, dtype)
    a = u[np.asarray(target, np.int64)]
    b = u[np.asarray(source, np.int64)]
    c = (a * b).sum(1) * dtype(EPS_SCALE)
    theta = np.arccos(c)
    ph = theta[:, None] * freqs[None, :]
    out = np.empty((len(c), 1 + 2 * len(freqs)), dtype)
    out[:, 0] = dtype(2.0 ** -0.5)
    out[:, 1:1 + len(freqs)] = np.sin(ph)
    out[:, 1 + len(freqs):] = np.cos(ph)
    return out / dtype(scale)


def fourier_basis_vjp(gout, u, target, source, freqs, scale) -> np.ndarray:
    """grad_unit [E, 3] in float64 (sums in row order, target terms then source terms, the
    reference's ordered form)."""
    u = np.asarray(u, np.float64)
    g = np.asarray(gout, np.float64)
    freqs = np.asarray(freqs, np.float64)
    nf = len(freqs)
    target = np.asarray(target, np.int64)
    source = np.asarray(source, np.int64)
    a, b = u[target], u[source]
    c = (a * b).sum(1) * EPS_SCALE
    theta = np.arccos(c)
    ph = theta[:, None] * freqs[None, :]
    dth = ((g[:, 1:1 + nf] * np.cos(ph) - g[:, 1 + nf:] * np.sin(ph)) * freqs).sum(1) / scale
    d = -dth / np.sqrt(np.maximum(1.0 - c * c, 1.0e-24)) * EPS_SCALE
    gu = np.zeros_like(u)
    np.add.at(gu, target, d[:, None] * b)
    np.add.at(gu, source, d[:, None] * a)
    return gu
