"""Stress of the engine-owned derivative (fastmd/engine/energy_derivative.py:110-140: a symmetric
strain of positions and cell, stress = dE/d(strain) / V): the FP64 oracle pinned on the CPU by
central finite differences of the energy under strain and, for the Morse pair potential, by the
closed-form pair virial; the HIP path (the virial of each model's edge-vector gradient) against
the oracle on a sheared, rotated cell (GPU), its energy and forces bitwise those of the "ef"
task."""
import types

import numpy as np
import pytest
import torch

from oracle import models as om
from fastmd_amd import systems

import test_models as tm
import test_threebody_model as ttb


def _system(n_cells=2):
    """A perovskite displaced from its sites (sizeable forces and shear stress) in a sheared cell
    rotated as a whole: no zero cell entries, no axis along x, y or z."""
    return tm._triclinic_rotated(systems.perovskite(n_cells, sigma=0.2))


def _oracle_fn(name, s, cutoff=6.0):
    """``fn(positions, cell) -> per-atom energies`` of the oracle model over the oracle's edge list
    of ``s`` at ``cutoff`` (the models keep only r < their own cutoff), and the wrapped positions."""
    center, neighbor, images, pos = tm._edges(s, cutoff=cutoff)
    if name == "morse":
        return (lambda p, c: om.morse_node_energy(p, c, center, neighbor, images)), pos
    if name == "mace_like":
        _, params, cfg, elem_of = tm._mace_params(128)
        elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
        return (lambda p, c: om.mace_like_node_energy(params, cfg, p, c, elem, center, neighbor, images)), pos
    _, params, cfg, elem_of = ttb._params(3.5)
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    return (lambda p, c: om.threebody_like_node_energy(params, cfg, p, c, elem, center, neighbor, images)), pos


# ------------------------------------------------------------------------------------ CPU pins
@pytest.mark.parametrize("name", ["morse", "mace_like", "threebody"])
def test_oracle_stress_is_the_strain_derivative(name):
    """Each component of the oracle's stress equals the central difference (h = 1e-6) of the FP64
    energy of the strained system, positions and cell deformed as x -> x (I + S), S = (e + e^T)/2
    with one entry of e set, divided by the volume; the tensor is symmetric and has shear parts.
    (Morse's edge list reaches 6.5 A: its potential is shifted in value only, so pairs that cross
    the cutoff under strain must be present on both sides.)"""
    s = _system()
    fn, pos = _oracle_fn(name, s, cutoff=6.5 if name == "morse" else 6.0)
    cell = torch.tensor(s.cell)
    e, f, stress = om.energy_forces_stress(fn, pos, cell)
    e_plain, f_plain, _ = om.energy_and_forces(lambda p: fn(p, cell), pos)
    assert float(abs(e - e_plain)) < 1e-10 and torch.allclose(f, f_plain, rtol=0, atol=1e-12)
    vol = abs(np.linalg.det(s.cell))
    h = 1e-6
    fd = np.zeros((3, 3))
    for a in range(3):
        for b in range(3):
            ends = []
            for sign in (1.0, -1.0):
                eps = torch.zeros(3, 3, dtype=torch.float64)
                eps[a, b] = sign * h
                sym = 0.5 * (eps + eps.T)
                ends.append(float(fn(pos + pos @ sym, cell + cell @ sym).sum()))
            fd[a, b] = (ends[0] - ends[1]) / (2 * h) / vol
    st = stress.numpy()
    assert np.abs(fd - st).max() < 1e-7 * np.abs(st).max()
    assert np.array_equal(st, st.T)
    off_diagonal = st[~np.eye(3, dtype=bool)]
    assert np.abs(off_diagonal).max() > 1e-3 * np.abs(st).max()


def test_oracle_morse_stress_is_the_pair_virial():
    """For a pair potential with E_i = 1/2 sum_j V(r_ij) the stress is the pair virial
    (1 / V) sum over ordered pairs of 1/2 V'(r) v v^T / r, V'(r) = 2 D a (1 - x) x with
    x = exp(-a (r - r0))."""
    s = _system()
    fn, pos = _oracle_fn("morse", s)
    _, _, stress = om.energy_forces_stress(fn, pos, torch.tensor(s.cell))
    center, neighbor, images, _ = tm._edges(s)
    v = (pos[neighbor] + images.double() @ torch.tensor(s.cell)) - pos[center]
    r = v.norm(dim=1)
    D, a, r0 = 0.3, 1.5, 3.0
    x = torch.exp(-a * (r - r0))
    dv = 2 * D * a * (1 - x) * x
    virial = (0.5 * dv / r)[:, None, None] * v[:, :, None] * v[:, None, :]
    expected = virial.sum(0) / abs(np.linalg.det(s.cell))
    assert torch.allclose(stress, expected, rtol=1e-12, atol=1e-15)


def test_engine_stress_contract_refusals():
    """The engine derivative forms stress for one system per batch: replica or system segments,
    a row subset and a model without a stress tap are refused before any kernel runs."""
    from fastmd_amd.engine.energy_derivative import EnergyDerivative

    class Tapped:
        name = "tapped"

        def node_energy(self, inputs, positions, cell):
            raise AssertionError("not reached")

        def energy_forces_stress(self, inputs, positions, cell):
            raise AssertionError("not reached")

    class Untapped:
        name = "untapped"

        def node_energy(self, inputs, positions, cell):
            raise AssertionError("not reached")

    batch = types.SimpleNamespace(positions=torch.zeros(8, 3), cell=torch.eye(3), systems=None)
    with pytest.raises(NotImplementedError, match="stress tap"):
        EnergyDerivative(Untapped())(batch, None, task="efs")
    with pytest.raises(NotImplementedError, match="one system"):
        EnergyDerivative(Tapped(), segments=2)(batch, None, task="efs")
    with pytest.raises(NotImplementedError, match="subset"):
        EnergyDerivative(Tapped())(batch, None, task="efs", n_real=6)


# ------------------------------------------------------------------------------------ GPU parity
def _gpu_adapter(name, device):
    if name == "morse":
        from fastmd_amd.models.pair_potential import MorsePairAdapter

        return MorsePairAdapter(device=device)
    if name == "mace_like":
        from fastmd_amd.models.mace_like import MaceLikeAdapter

        return MaceLikeAdapter(tm._mace_params(128)[0], device=device)
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter

    return ThreeBodyAdapter(ttb._params(3.5)[0], device=device)


@pytest.mark.gpu
@pytest.mark.parametrize("name,n_cells", [("morse", 3), ("mace_like", 3), ("threebody", 3), ("mace_like", (6, 6, 6))])
def test_stress_gpu_matches_oracle(device, name, n_cells):
    """The "efs" task through the fixed-capacity builder (padding rows present) on a sheared,
    rotated cell: stress within 1e-5 of the largest component of the FP64 oracle's (the float32
    edge gradients summed in float64; measured 2e-7 .. 4e-7 of it), symmetric, bitwise
    reproducible; energy and forces bitwise those of the "ef" task."""
    from fastmd_amd.engine.energy_derivative import EnergyDerivative

    print(f"[stress] {name} cells={n_cells}", flush=True)
    s = _system(n_cells)
    n = s.n_atoms
    adapter = _gpu_adapter(name, device)
    if name == "threebody":
        builder = ttb._builder(s, 3.5, device)
    else:
        builder = tm._gpu_builder(s, int(n * 18 / 2) + 100, device)
    _, status = builder.build(torch.tensor(s.positions, device=device))
    assert not bool(status.overflow.item())
    inputs = adapter.prepare(builder.batch)
    deriv = EnergyDerivative(adapter)
    out = deriv(builder.batch, inputs, task="efs", n_real=n)
    again = deriv(builder.batch, inputs, task="efs", n_real=n)
    plain = deriv(builder.batch, inputs, task="ef", n_real=n)
    torch.cuda.synchronize()
    stress = out["s"][0]
    assert stress.shape == (3, 3) and stress.dtype == torch.float32
    assert torch.equal(stress, again["s"][0]) and torch.equal(stress, stress.T)
    assert torch.equal(out["e"], plain["e"]) and torch.equal(out["f"][0], plain["f"][0])
    fn, pos = _oracle_fn(name, s, cutoff=6.5 if name == "morse" else 6.0)
    _, _, ref = om.energy_forces_stress(fn, pos, torch.tensor(s.cell))
    err = float((stress.cpu().double() - ref).abs().max())
    scale = float(ref.abs().max())
    print(f"[stress] {name} cells={n_cells}: max|s| {scale:.3e} eV/A^3, max err {err:.3e}", flush=True)
    assert err < 1e-5 * scale
