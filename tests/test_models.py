"""Models on the HIP kernels (MACE-like, Morse) vs the PyTorch-CPU oracle; the oracle pinned by
finite differences, Newton's third law and exact-zero padding (CPU)."""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import models as om
from oracle import nl as onl
from fastmd_amd import systems

F32 = np.float32


def _edges(s, cutoff=6.0, jitter_seed=None):
    cell32 = s.cell.astype(F32)
    inv = np.linalg.inv(cell32.astype(np.float64)).astype(F32)
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    cand = onl.candidates(wrapped, cell32, F32((cutoff + 1.0) ** 2), 1504)
    b = onl.build(s.positions, inv, cell32, cand, s.positions.astype(F32), wraps, F32(cutoff ** 2), F32(2.0),
                  (1, 0, 0), 10 ** 7)
    e = b.n_edges
    return (torch.tensor(b.center[:e].astype(np.int64)), torch.tensor(b.neighbor[:e].astype(np.int64)),
            torch.tensor(b.images[:e]), torch.tensor(b.wrapped.astype(np.float64)))


def _mace_params(channels=128):
    from fastmd_amd.models.mace_like import MaceLike, MaceLikeConfig

    cfg = MaceLikeConfig(channels=channels)
    m = MaceLike(cfg)
    params = {k: v.detach().clone() for k, v in m.named_parameters()}
    elem_of = {z: k for k, z in enumerate(cfg.elements)}
    return m, params, dataclasses.asdict(cfg), elem_of


def _mace_fn(params, cfg, elem, center, neighbor, images, cell):
    return lambda pos: om.mace_like_node_energy(params, cfg, pos, cell, elem, center, neighbor, images)


# ------------------------------------------------------------------------------------ CPU pins
def test_mace_like_oracle_forces_are_the_energy_gradient():
    s = systems.perovskite(2)
    center, neighbor, images, pos = _edges(s)
    _, params, cfg, elem_of = _mace_params(64)
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    cell = torch.tensor(s.cell)
    fn = _mace_fn(params, cfg, elem, center, neighbor, images, cell)
    e, f, _ = om.energy_and_forces(fn, pos)
    assert float(f.abs().max()) > 1e-3  # the model is not trivial
    rng = np.random.default_rng(0)
    for atom in rng.choice(pos.shape[0], 4, replace=False):
        for k in range(3):
            h = 1e-5
            dp = torch.zeros_like(pos)
            dp[atom, k] = h
            fd = -(fn(pos + dp).sum() - fn(pos - dp).sum()) / (2 * h)
            assert abs(float(fd) - float(f[atom, k])) < 1e-6 * max(1.0, abs(float(fd)))
    assert float(f.sum(0).abs().max()) < 1e-10  # Newton's third law (periodic, translation invariant)
    e_shift, _, _ = om.energy_and_forces(fn, pos + torch.tensor([0.3, -0.2, 0.1], dtype=torch.float64))
    assert abs(float(e_shift - e)) < 1e-9 * abs(float(e))


def test_mace_like_oracle_padding_adds_exactly_nothing():
    s = systems.perovskite(2)
    center, neighbor, images, pos = _edges(s)
    _, params, cfg, elem_of = _mace_params(64)
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    cell = torch.tensor(s.cell)
    n = pos.shape[0]
    pad = torch.arange(50) % n
    c2 = torch.cat([center, pad])
    n2 = torch.cat([neighbor, pad])
    i2 = torch.cat([images, torch.tensor([[1, 0, 0]] * 50, dtype=images.dtype)])
    e1, f1, _ = om.energy_and_forces(_mace_fn(params, cfg, elem, center, neighbor, images, cell), pos)
    e2, f2, _ = om.energy_and_forces(_mace_fn(params, cfg, elem, c2, n2, i2, cell), pos)
    assert float(e1) == float(e2)
    assert torch.equal(f1, f2)


def test_morse_oracle_dimer_closed_form_and_gradient():
    cell = torch.eye(3, dtype=torch.float64) * 30.0
    pos = torch.tensor([[0.0, 0.0, 0.0], [3.5, 0.0, 0.0]], dtype=torch.float64)
    center, neighbor = torch.tensor([0, 1]), torch.tensor([1, 0])
    images = torch.zeros(2, 3, dtype=torch.int32)
    e, f, node = om.energy_and_forces(om.morse_node_energy, pos, cell, center, neighbor, images)
    D, a, r0, rc = 0.3, 1.5, 3.0, 6.0
    v = lambda r: D * ((1 - np.exp(-a * (r - r0))) ** 2 - 1) - D * ((1 - np.exp(-a * (rc - r0))) ** 2 - 1)
    assert float(e) == pytest.approx(v(3.5), rel=1e-12)
    dv = 2 * D * (1 - np.exp(-a * 0.5)) * a * np.exp(-a * 0.5)
    assert float(f[1, 0]) == pytest.approx(-dv, rel=1e-10) and float(f[0, 0]) == pytest.approx(dv, rel=1e-10)


# ------------------------------------------------------------------------------------ GPU parity
def _gpu_builder(s, u_cap, device):
    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    return FixedCapacityGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers),
                                     u_capacity=u_cap, atom_graph_cutoff=6.0, candidate_cutoff=8.0, device=device)


@pytest.mark.gpu
@pytest.mark.parametrize("n_cells,channels,hoist,fused", [
    (3, 128, None, True), (3, 64, None, True), (3, 256, None, True), ((6, 6, 6), 128, None, True),
    (3, 64, 0, True), (3, 128, 0, True), (3, 256, 0, True), ((6, 6, 6), 128, 10 ** 9, True),
    (3, 64, None, False), (3, 128, None, False), (3, 256, None, False), ((6, 6, 6), 128, None, False),
    ((10, 10, 10), 128, None, False)])
def test_mace_like_gpu_matches_oracle(device, n_cells, channels, hoist, fused, monkeypatch):
    """Energies within 1e-5 eV/atom and forces within 1e-4 eV/A of the FP64 oracle, through the
    fixed-capacity builder (padding rows present), bitwise reproducible. ``hoist`` overrides the
    edge-list size from which the receiver block of the edge GEMM is formed per atom (0: always,
    10**9: never), so both evaluation orders of z are checked at every width; ``fused`` selects the
    fused node kernels or the unfused chain of GEMMs and contraction kernels; at 5 000 atoms the
    unfused node GEMMs take their split-plane grouped form."""
    from fastmd_amd.engine.energy_derivative import EnergyDerivative
    from fastmd_amd.models import mace_like
    from fastmd_amd.models.mace_like import MaceLikeAdapter

    if hoist is not None:
        monkeypatch.setattr(mace_like, "HOIST_MIN_ROWS", hoist)
    monkeypatch.setattr(mace_like, "FUSED_NODE", fused)
    print(f"[mace] cells={n_cells} C={channels} hoist={hoist} fused={fused}", flush=True)
    s = systems.perovskite(n_cells, sigma=0.2)  # displaced from the symmetric sites: sizeable forces
    n = s.n_atoms
    m, params, cfg, elem_of = _mace_params(channels)
    adapter = MaceLikeAdapter(m, device=device)
    builder = _gpu_builder(s, int(n * 18 / 2) + 100, device)
    builder.refresh_candidates(torch.tensor(s.positions, device=device))
    graph, status = builder.build(torch.tensor(s.positions, device=device), rebuild_candidates=False)
    inputs = adapter.prepare(builder.batch)
    deriv = EnergyDerivative(adapter)
    out = deriv(builder.batch, inputs, n_real=n)
    out2 = deriv(builder.batch, inputs, n_real=n)
    torch.cuda.synchronize()
    assert int(status.edge_count.item()) < builder.e_capacity and not bool(status.overflow.item())
    e_gpu = float(out["e"].item())
    f_gpu = out["f"][0].cpu().double()
    assert torch.equal(out["e"], out2["e"])  # deterministic
    assert torch.equal(out["f"][0], out2["f"][0])
    center, neighbor, images, pos = _edges(s)
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    e_ref, f_ref, _ = om.energy_and_forces(
        _mace_fn(params, cfg, elem, center, neighbor, images, torch.tensor(s.cell)), pos)
    assert abs(e_gpu - float(e_ref)) / n < 1e-5
    assert float((f_gpu - f_ref).abs().max()) < 1e-4
    assert float(f_ref.abs().max()) > 1e-2
    assert float((f_gpu - f_ref).abs().max()) / float(f_ref.abs().max()) < 1e-4
    # the engine takes the adapter's explicit VJP; the autograd route over node_energy (the
    # reference engine's route) runs the same kernels and gives the same bits
    with torch.enable_grad():
        leaf = builder.batch.positions.detach().requires_grad_(True)
        from fastmd_amd.engine.energy_derivative import sum_f64

        energy = sum_f64(adapter.node_energy(inputs, leaf, builder.batch.cell)[:n])
        (grad,) = torch.autograd.grad(energy, (leaf,))
    assert torch.equal(energy.detach().reshape(1), out["e"])
    assert torch.equal(-grad, out["f"][0])


@pytest.mark.gpu
def test_morse_gpu_matches_oracle(device):
    from fastmd_amd.engine.energy_derivative import EnergyDerivative
    from fastmd_amd.models.pair_potential import MorsePairAdapter

    s = systems.perovskite(3, sigma=0.2)
    adapter = MorsePairAdapter(device=device)
    builder = _gpu_builder(s, 1300, device)
    _, status = builder.build(torch.tensor(s.positions, device=device))
    assert not bool(status.overflow.item())
    out = EnergyDerivative(adapter)(builder.batch, adapter.prepare(builder.batch), n_real=s.n_atoms)
    center, neighbor, images, pos = _edges(s)
    e_ref, f_ref, _ = om.energy_and_forces(om.morse_node_energy, pos, torch.tensor(s.cell), center, neighbor, images)
    assert abs(float(out["e"].item()) - float(e_ref)) / s.n_atoms < 1e-5
    assert float((out["f"][0].cpu().double() - f_ref).abs().max()) < 1e-4
