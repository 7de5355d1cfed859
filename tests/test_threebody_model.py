"""The three-body (CHGNet/MatRIS-style) model: the FP64 oracle pinned by finite differences,
invariances, the brute-force triplet set and smoothness at the bond cutoff (CPU); the HIP model
(line-graph builder, Fourier basis, gated sums, explicit VJP) against the oracle (GPU)."""
import dataclasses
import math

import numpy as np
import pytest
import torch

from oracle import models as om
from oracle import nl as onl
from fastmd_amd import systems
from fastmd_amd.adapters.protocol import PaddingRule

F32 = np.float32


def _edges(s, cutoff=6.0):
    cell32 = s.cell.astype(F32)
    inv = np.linalg.inv(cell32.astype(np.float64)).astype(F32)
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    cand = onl.candidates(wrapped, cell32, F32((cutoff + 1.0) ** 2), 1504)
    b = onl.build(s.positions, inv, cell32, cand, s.positions.astype(F32), wraps, F32(cutoff ** 2), F32(2.0),
                  (1, 0, 0), 10 ** 7)
    e = b.n_edges
    return (torch.tensor(b.center[:e].astype(np.int64)), torch.tensor(b.neighbor[:e].astype(np.int64)),
            torch.tensor(b.images[:e]), torch.tensor(b.wrapped.astype(np.float64)))


def _params(bond_cutoff=3.5, channels=64):
    from fastmd_amd.models.threebody_like import ThreeBodyConfig, ThreeBodyLike

    cfg = ThreeBodyConfig(channels=channels, bond_cutoff=bond_cutoff)
    m = ThreeBodyLike(cfg)
    params = {k: v.detach().clone() for k, v in m.named_parameters()}
    elem_of = {z: k for k, z in enumerate(cfg.elements)}
    return m, params, dataclasses.asdict(cfg), elem_of


def _fn(params, cfg, s, edges, bond_rows=None, cell=None):
    center, neighbor, images, _ = edges
    elem_of = {z: k for k, z in enumerate(cfg["elements"])}
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    cell = torch.tensor(s.cell) if cell is None else cell
    return lambda pos: om.threebody_like_node_energy(params, cfg, pos, cell, elem, center, neighbor, images,
                                                     bond_rows=bond_rows)


# ------------------------------------------------------------------------------------ CPU pins
def test_oracle_forces_gradient_newton_translation():
    s = systems.perovskite(2, sigma=0.2)
    edges = _edges(s)
    _, params, cfg, _ = _params(3.5)
    fn = _fn(params, cfg, s, edges)
    pos = edges[3]
    e, f, _ = om.energy_and_forces(fn, pos)
    assert float(f.abs().max()) > 1e-3
    rng = np.random.default_rng(0)
    for atom in rng.choice(pos.shape[0], 4, replace=False):
        for k in range(3):
            h = 1e-5
            dp = torch.zeros_like(pos)
            dp[atom, k] = h
            fd = -(fn(pos + dp).sum() - fn(pos - dp).sum()) / (2 * h)
            assert abs(float(fd) - float(f[atom, k])) < 1e-6 * max(1.0, abs(float(fd)))
    assert float(f.sum(0).abs().max()) < 1e-10
    e_shift, _, _ = om.energy_and_forces(fn, pos + torch.tensor([0.3, -0.2, 0.1], dtype=torch.float64))
    assert abs(float(e_shift - e)) < 1e-9 * abs(float(e))


def test_oracle_rotation_invariance_and_three_body_terms_present():
    """A common rotation of positions and cell leaves the energy unchanged (the angle basis sees
    only bond angles); the three-body update changes it (triplets exist at 3.5 A, not at 1 A)."""
    s = systems.perovskite(2, sigma=0.2)
    edges = _edges(s)
    _, params, cfg, _ = _params(3.5)
    pos = edges[3]
    q, r = np.linalg.qr(np.random.default_rng(4).normal(size=(3, 3)))
    rot = torch.tensor(q * np.sign(np.diag(r)))
    e = om.threebody_like_node_energy(params, cfg, pos, torch.tensor(s.cell), torch.tensor(
        [{55: 0, 50: 1, 53: 2}[int(z)] for z in s.numbers]), *edges[:3]).sum()
    e_rot = om.threebody_like_node_energy(params, cfg, pos @ rot.T, torch.tensor(s.cell) @ rot.T, torch.tensor(
        [{55: 0, 50: 1, 53: 2}[int(z)] for z in s.numbers]), *edges[:3]).sum()
    assert abs(float(e - e_rot)) < 1e-10 * abs(float(e))
    none = dict(cfg, bond_cutoff=1.0)
    e_none = _fn(params, none, s, edges)(pos).sum()
    assert abs(float(e - e_none)) > 1e-4
    # no bonds: the energy does not depend on the angle weights at all
    p2 = {k: (v * 3.0 if k.endswith("W3") else v) for k, v in params.items()}
    assert float(_fn(p2, none, s, edges)(pos).sum()) == float(e_none)


def test_oracle_triplets_match_brute_force_set():
    s = systems.perovskite(2, sigma=0.2)
    center, neighbor, images, pos = _edges(s)
    vec = om.edge_vectors(pos, torch.tensor(s.cell), center, neighbor, images)
    short = (vec.norm(dim=1) < 3.5).numpy()
    bonds = torch.nonzero(torch.tensor(short)).flatten()
    atom, b1, b2 = om.triplets_of(center, bonds)
    got = {(int(a), (int(neighbor[x]), *map(int, images[x])), (int(neighbor[y]), *map(int, images[y])))
           for a, x, y in zip(atom, b1, b2)}
    assert len(got) == len(atom) > 0
    assert got == onl.triplet_set(center.numpy(), neighbor.numpy(), images.numpy(), short, len(center))


def test_oracle_smooth_at_the_bond_cutoff():
    """The envelope is C2 at rb: the energy along a path that takes bonds across rb has no jump
    in value or slope (central slopes just inside and outside agree)."""
    s = systems.perovskite(2, sigma=0.0)
    edges = _edges(s)
    _, params, cfg, _ = _params(3.1)  # the B-X bonds (3.1 A) sit at the bond cutoff
    fn = _fn(params, cfg, s, edges)
    pos = edges[3]
    d = torch.zeros_like(pos)
    d[1, 0] = 1.0  # move the first B site along x: its +x and -x bonds cross 3.1 A
    energy = lambda t: float(fn(pos + t * d).sum())  # noqa: E731
    h = 1e-4
    for t0 in (-1e-3, 1e-3):
        slope_l = (energy(t0) - energy(t0 - h)) / h
        slope_r = (energy(t0 + h) - energy(t0)) / h
        assert abs(slope_l - slope_r) < 1e-4 * max(1.0, abs(slope_l))
    assert abs(energy(1e-6) - energy(-1e-6)) < 1e-8


# ------------------------------------------------------------------------------------ GPU parity
def _builder(s, bond_cutoff, device, u_cap=None, t_cap=None):
    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    n = s.n_atoms
    return FixedCapacityGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers),
                                     u_capacity=u_cap or int(n * 18 / 2) + 100, t_capacity=t_cap or 40 * n,
                                     atom_graph_cutoff=6.0, line_graph_cutoff=bond_cutoff, candidate_cutoff=8.0,
                                     padding=PaddingRule("far_self_loops"), device=device)


@pytest.mark.gpu
@pytest.mark.parametrize("n_cells,bond_cutoff", [(3, 3.5), (3, 3.0), ((6, 6, 6), 3.5), ((6, 6, 6), 3.0),
                                                 (10, 3.5), (10, 3.0)])
def test_threebody_gpu_matches_oracle(device, n_cells, bond_cutoff):
    """Energies within 1e-5 eV/atom and forces within 1e-4 eV/A of the FP64 oracle through the
    line-graph builder (padding pairs and triplets present); bitwise reproducible; the autograd
    route over node_energy gives the explicit VJP's bits."""
    from fastmd_amd.engine.energy_derivative import EnergyDerivative, sum_f64
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter

    print(f"[threebody] cells={n_cells} rb={bond_cutoff}", flush=True)
    s = systems.perovskite(n_cells, sigma=0.2)
    n = s.n_atoms
    m, params, cfg, _ = _params(bond_cutoff)
    adapter = ThreeBodyAdapter(m, device=device)
    builder = _builder(s, bond_cutoff, device)
    graph, status = builder.build(torch.tensor(s.positions, device=device))
    assert not bool(status.overflow.item())
    inputs = adapter.prepare(builder.batch)
    deriv = EnergyDerivative(adapter)
    out = deriv(builder.batch, inputs, n_real=n)
    out2 = deriv(builder.batch, inputs, n_real=n)
    torch.cuda.synchronize()
    assert torch.equal(out["e"], out2["e"]) and torch.equal(out["f"][0], out2["f"][0])
    e_gpu, f_gpu = float(out["e"].item()), out["f"][0].cpu().double()
    edges = _edges(s)
    n_edges = len(edges[0])
    assert int(builder.edge_offsets[-1].item()) == n_edges
    bonds = torch.nonzero(builder.short_flags[:n_edges].cpu().bool()).flatten()
    t_real = int(builder.pair_offsets[-1].item())
    print(f"[threebody] edges={n_edges} bonds={len(bonds)} triplets={t_real}", flush=True)
    e_ref, f_ref, _ = om.energy_and_forces(_fn(params, cfg, s, edges, bond_rows=bonds), edges[3])
    assert abs(e_gpu - float(e_ref)) / n < 1e-5
    assert float(f_ref.abs().max()) > 1e-2
    assert float((f_gpu - f_ref).abs().max()) < 1e-4
    with torch.enable_grad():
        leaf = builder.batch.positions.detach().requires_grad_(True)
        energy = sum_f64(adapter.node_energy(inputs, leaf, builder.batch.cell)[:n])
        (grad,) = torch.autograd.grad(energy, (leaf,))
    assert torch.equal(energy.detach().reshape(1), out["e"])
    assert torch.equal(-grad, out["f"][0])


@pytest.mark.gpu
@pytest.mark.parametrize("channels", [128, 192, 256])
def test_threebody_gpu_channels_match_oracle(device, channels):
    """Channel counts that give the segment and bond kernels two, three and four channels per lane:
    energies within 1e-5 eV/atom and forces within 1e-4 eV/A of the FP64 oracle on the 135-atom
    perovskite at 3.5 A."""
    from fastmd_amd.engine.energy_derivative import EnergyDerivative
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter

    print(f"[threebody] channels={channels}", flush=True)
    s = systems.perovskite(3, sigma=0.2)
    n = s.n_atoms
    m, params, cfg, _ = _params(3.5, channels=channels)
    adapter = ThreeBodyAdapter(m, device=device)
    builder = _builder(s, 3.5, device)
    builder.build(torch.tensor(s.positions, device=device))
    inputs = adapter.prepare(builder.batch)
    out = EnergyDerivative(adapter)(builder.batch, inputs, n_real=n)
    torch.cuda.synchronize()
    edges = _edges(s)
    bonds = torch.nonzero(builder.short_flags[:len(edges[0])].cpu().bool()).flatten()
    assert int(builder.pair_offsets[-1].item()) > 0
    e_ref, f_ref, _ = om.energy_and_forces(_fn(params, cfg, s, edges, bond_rows=bonds), edges[3])
    assert abs(float(out["e"].item()) - float(e_ref)) / n < 1e-5
    assert float((out["f"][0].cpu().double() - f_ref).abs().max()) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("two_index,C,max_run", [(False, 128, 12), (True, 128, 12), (False, 100, 40),
                                                 (True, 40, 40), (False, 256, 20)])
def test_gated_segment_sum_and_vjp(device, two_index, C, max_run):
    """fmd_tb_gated_sum_f32 / _bwd_f32 (both weight forms) against float64 torch: the sums, the
    pre-activation and weight gradients, the per-segment gradient sums; rows past the last run
    get zero gradients. Channel counts below and between multiples of 64 (lanes past C idle) and
    runs longer than one batch of rows."""
    from fastmd_amd import _abi

    gen = torch.Generator().manual_seed(3)
    rows, n_seg, nw = 400 * max_run // 2 + 600, 400, 500
    counts = torch.randint(0, max_run, (n_seg,), generator=gen)
    off = torch.zeros(n_seg + 1, dtype=torch.int64)
    off[1:] = torch.cumsum(counts, 0)
    used = int(off[-1])
    assert used < rows
    z = torch.randn(rows, C, generator=gen)
    w = torch.rand(nw, 2, generator=gen)  # column 0 is the weight, stride 2
    idx = torch.randint(0, nw, (rows, 3), generator=gen, dtype=torch.int32)
    g = torch.randn(n_seg, C, generator=gen)
    scale = 0.37
    seg = torch.repeat_interleave(torch.arange(n_seg), counts)
    z64 = z[:used].double().requires_grad_(True)
    w64 = w[:, 0].double().requires_grad_(True)
    wr = w64[idx[:used, 0].long()] * (w64[idx[:used, 2].long()] if two_index else 1.0)
    out64 = torch.zeros(n_seg, C, dtype=torch.float64).index_add(
        0, seg, torch.nn.functional.silu(z64) * wr[:, None]) * scale
    (out64 * g.double()).sum().backward()
    zd, wd, idd, offd, gd = (t.to(device) for t in (z, w, idx, off, g))
    out = torch.full((n_seg, C), 1.5, device=device)
    i2 = idd[:, 2].data_ptr() if two_index else None
    _abi.call("fmd_tb_gated_sum_f32", zd.data_ptr(), C, rows, C, wd.data_ptr(), 2, idd[:, 0].data_ptr(), i2, 3,
              offd.data_ptr(), n_seg, scale, out.data_ptr(), C, 1, _abi.stream_handle())
    gz = torch.full((rows, C), 7.0, device=device)
    gsum = torch.empty(n_seg, C, device=device)
    gw = torch.full((rows, 2), 9.0, device=device)
    _abi.call("fmd_tb_gated_sum_bwd_f32", gd.data_ptr(), C, zd.data_ptr(), C, rows, C, wd.data_ptr(), 2,
              idd[:, 0].data_ptr(), i2, 3, offd.data_ptr(), n_seg, scale, gz.data_ptr(), C, gsum.data_ptr(), C,
              gw.data_ptr(), 2, 0, _abi.stream_handle())
    torch.cuda.synchronize()
    assert torch.allclose(out.cpu().double() - 1.5, out64.detach(), atol=1e-5, rtol=1e-5)
    assert torch.allclose(gz[:used].cpu().double(), z64.grad, atol=1e-5, rtol=1e-5)
    assert not gz[used:].any()
    assert torch.allclose(gsum.cpu().double(), torch.zeros(n_seg, C, dtype=torch.float64).index_add(
        0, seg, z64.grad), atol=1e-4, rtol=1e-5)
    # the weight's gradient from its per-row terms
    silu_g = (torch.nn.functional.silu(z64.detach()) * (g.double() * scale)[seg]).sum(1)
    if two_index:
        a, b = w64.detach()[idx[:used, 0].long()], w64.detach()[idx[:used, 2].long()]
        assert torch.allclose(gw[:used, 0].cpu().double(), silu_g * b, atol=1e-4, rtol=1e-5)
        assert torch.allclose(gw[:used, 1].cpu().double(), silu_g * a, atol=1e-4, rtol=1e-5)
        assert not gw[used:].any()
    else:
        assert torch.allclose(gw[:used, 0].cpu().double(), silu_g, atol=1e-4, rtol=1e-5)
        assert not gw[used:, 0].any()
    gw_total = torch.zeros(nw, dtype=torch.float64)
    gw_total.index_add_(0, idx[:used, 0].long(), gw[:used, 0].cpu().double())
    if two_index:
        gw_total.index_add_(0, idx[:used, 2].long(), gw[:used, 1].cpu().double())
    assert torch.allclose(gw_total, w64.grad, atol=1e-3, rtol=1e-5)
