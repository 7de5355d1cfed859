"""Models on the HIP kernels (MACE-like, Morse) vs the PyTorch-CPU oracle (GPU, also on a rotated
triclinic cell and at the 10 000-atom headline size); the oracle pinned on the CPU by finite
differences, Newton's third law, exact-zero padding, rotation invariance with forces rotating,
atom-permutation invariance, zero forces at inversion centres and a hand-reduced dimer closed
form of the two-layer model."""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import models as om
from oracle import nl as onl
from fastmd_amd import systems
from fastmd_amd.adapters.protocol import PaddingRule

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


def _rotation(seed):
    """A random proper rotation (det +1) from the QR of a seeded Gaussian matrix."""
    q, r = np.linalg.qr(np.random.default_rng(seed).normal(size=(3, 3)))
    q = q * np.sign(np.diag(r))
    if np.linalg.det(q) < 0:
        q[:, 0] = -q[:, 0]
    return q


def _triclinic_rotated(s, seed=7, shear=(0.12, -0.08, 0.05)):
    """The same crystal (fractional coordinates kept) in a sheared cell, b' = b + s0 a and
    c' = c + s1 a + s2 b, then rotated as a whole by a random rotation: a general cell matrix
    with no zero entries and no axis along x, y or z."""
    frac = s.positions @ np.linalg.inv(s.cell)
    shear_m = np.array([[1.0, 0.0, 0.0], [shear[0], 1.0, 0.0], [shear[1], shear[2], 1.0]])
    cell = (shear_m @ s.cell) @ _rotation(seed).T
    return systems.System(frac @ cell, cell, s.numbers.copy(), s.masses.copy())


def test_mace_like_oracle_rotation_invariant_and_forces_rotate():
    """A common rotation R of the positions and of a triclinic cell (same edges and images)
    leaves every per-atom energy unchanged and rotates the forces, F' = F R^T: the model sees
    only lengths, u . h1 projections and |P1|^2, and carries h1 as a vector. A sign or index
    mistake in u, the projection or the vector message breaks the second property."""
    s = _triclinic_rotated(systems.perovskite(2, sigma=0.2), seed=3)
    center, neighbor, images, pos = _edges(s)
    _, params, cfg, elem_of = _mace_params(64)
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    cell = torch.tensor(s.cell)
    e, f, node = om.energy_and_forces(_mace_fn(params, cfg, elem, center, neighbor, images, cell), pos)
    assert float(f.abs().max()) > 1e-2
    for seed in (11, 12):
        rot = torch.tensor(_rotation(seed))
        e_r, f_r, node_r = om.energy_and_forces(
            _mace_fn(params, cfg, elem, center, neighbor, images, cell @ rot.T), pos @ rot.T)
        assert float((node_r - node).abs().max()) < 1e-12 * float(node.abs().max())
        assert abs(float(e_r - e)) < 1e-12 * abs(float(e))
        assert float((f_r - f @ rot.T).abs().max()) < 1e-10 * float(f.abs().max())


def test_mace_like_oracle_permutation_invariant():
    """Relabelling the atoms (and listing the edge rows in another order) permutes the per-atom
    energies and forces the same way and leaves the total unchanged."""
    s = systems.perovskite(2, sigma=0.2)
    center, neighbor, images, pos = _edges(s)
    _, params, cfg, elem_of = _mace_params(64)
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    cell = torch.tensor(s.cell)
    e, f, node = om.energy_and_forces(_mace_fn(params, cfg, elem, center, neighbor, images, cell), pos)
    rng = np.random.default_rng(5)
    perm = torch.tensor(rng.permutation(s.n_atoms))  # new atom k is old atom perm[k]
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(s.n_atoms)
    rows = torch.tensor(rng.permutation(center.shape[0]))
    fn_p = _mace_fn(params, cfg, elem[perm], inv[center[rows]], inv[neighbor[rows]], images[rows], cell)
    e_p, f_p, node_p = om.energy_and_forces(fn_p, pos[perm])
    assert abs(float(e_p - e)) < 1e-12 * abs(float(e))
    assert float((node_p - node[perm]).abs().max()) < 1e-12 * float(node.abs().max())
    assert float((f_p - f[perm]).abs().max()) < 1e-10 * float(f.abs().max())


def test_mace_like_oracle_symmetric_sites_have_zero_forces():
    """On the unjittered cubic perovskite every atom sits on an inversion centre, so every force
    vanishes (to rounding) while the energy does not."""
    s = systems.perovskite(2, sigma=0.0)
    center, neighbor, images, _ = _edges(s)
    pos = torch.tensor(s.positions)  # float64 sites (inside the cell, so no wrap): no float32 rounding
    _, params, cfg, elem_of = _mace_params(64)
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    e, f, _ = om.energy_and_forces(_mace_fn(params, cfg, elem, center, neighbor, images, torch.tensor(s.cell)), pos)
    assert abs(float(e)) > 1.0 and float(f.abs().max()) < 1e-11


def _np_silu(x):
    return x / (1.0 + np.exp(-x))


def _dimer_energy_closed_form(params, cfg, r, e_pair):
    """Total energy of an isolated dimer at separation r written out from the model's definition
    (per layer: gather-cat, edge GEMM, gated messages, contraction, node update; the readout), in
    NumPy with the geometry reduced by hand. Atom i's only edge comes from the other atom j, and
    u_1 = -u_0. Every vector feature stays parallel to the bond, h1_i = u_i (x) v_i, so
      h1_j . u_i = -v_j,   m1_i = u_i (x) (wb h0_j - wd v_j),   |P1_i|^2 = ((wb h0_j - wd v_j)/avg Wm1)^2
    and the model reduces to channel vectors only. Independent of the oracle's edge lists, index
    sums and 3-vectors."""
    p = {k: v.detach().double().numpy() for k, v in params.items()}
    C, nb, L, rc, avg = cfg["channels"], cfg["n_basis"], cfg["num_interactions"], cfg["cutoff"], cfg["avg_num_neighbors"]
    x = r / rc
    fcut = 1 - 21 * x ** 5 + 35 * x ** 6 - 15 * x ** 7 if x < 1 else 0.0
    n = np.arange(1, nb + 1)
    ef = np.sqrt(2.0 / rc) * np.sin(n * np.pi * r / rc) / r * fcut
    h = [p["embedding"][e_pair[0]], p["embedding"][e_pair[1]]]
    v = [np.zeros(C), np.zeros(C)]
    h_first = None
    for t in range(L):
        W = {k.split(".", 2)[2]: val for k, val in p.items() if k.startswith(f"layers.{t}.")}
        new_h, new_v = [], []
        for i in (0, 1):
            j = 1 - i
            z = np.concatenate([h[j], h[i], ef]) @ W["W1"]
            w = _np_silu(z) * fcut
            wa, wb, wc, wd = w[:C], w[C:2 * C], w[2 * C:3 * C], w[3 * C:]
            P0 = ((wa * h[j] - wc * v[j]) / avg) @ W["Wm0"]
            p1 = ((wb * h[j] - wd * v[j]) / avg) @ W["Wm1"]
            n1 = p1 * p1
            c = W["Wc"][e_pair[i]]
            B0 = c[0] * P0 + c[1] * P0 ** 2 + c[2] * n1 + c[3] * P0 ** 3 + c[4] * P0 * n1
            new_h.append(B0 @ W["Wo0"] + h[i] @ W["Wsc0"])
            d = W["Wd"][e_pair[i]]
            new_v.append(((d[0] + d[1] * P0 + d[2] * P0 ** 2 + d[3] * n1) * p1) @ W["Wo1"])
        if t == 0:
            h_first = new_h
        h, v = new_h, new_v
    total = 0.0
    for i in (0, 1):
        e_i = h_first[i] @ p["wr1"] + _np_silu(h[i] @ p["Wr2a"]) @ p["wr2b"]
        total += p["e0"][e_pair[i]] + cfg["scale"] * e_i + cfg["shift"]
    return total


@pytest.mark.parametrize("r", [2.7, 4.1, 5.5])
def test_mace_like_oracle_dimer_closed_form(r):
    """The oracle on an isolated, randomly oriented Cs-I dimer (two layers, so the vector
    features of the first layer feed the second) equals the hand-reduced closed form; its forces
    are equal and opposite, along the bond, and equal -dE/dr of the closed form."""
    _, params, cfg, elem_of = _mace_params(64)
    e_pair = (elem_of[55], elem_of[53])
    u = _rotation(9)[0]
    pos = torch.tensor(np.array([[11.0, 12.0, 13.0], [11.0, 12.0, 13.0] + r * u]))
    cell = torch.eye(3, dtype=torch.float64) * 40.0
    fn = _mace_fn(params, cfg, torch.tensor(e_pair), torch.tensor([0, 1]), torch.tensor([1, 0]),
                  torch.zeros(2, 3, dtype=torch.int32), cell)
    e, f, _ = om.energy_and_forces(fn, pos)
    closed = _dimer_energy_closed_form(params, cfg, r, e_pair)
    assert abs(float(e) - closed) < 1e-12 * abs(closed)
    h = 1e-5
    dedr = (_dimer_energy_closed_form(params, cfg, r + h, e_pair)
            - _dimer_energy_closed_form(params, cfg, r - h, e_pair)) / (2 * h)
    assert abs(dedr) > 1e-3
    f1 = f[1].numpy()
    assert np.abs(f1 + dedr * u).max() < 1e-7 * max(1.0, abs(dedr))
    assert np.abs(f[0].numpy() + f1).max() < 1e-12 * abs(dedr)
    # one layer only: the vector features never enter, and the closed form still holds
    cfg1 = dict(cfg, num_interactions=1)
    p1 = {k: v for k, v in params.items() if not k.startswith("layers.1.")}
    fn1 = _mace_fn(p1, cfg1, torch.tensor(e_pair), torch.tensor([0, 1]), torch.tensor([1, 0]),
                   torch.zeros(2, 3, dtype=torch.int32), cell)
    assert abs(float(fn1(pos).sum()) - _dimer_energy_closed_form(p1, cfg1, r, e_pair)) < 1e-12 * abs(closed)


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
                                     u_capacity=u_cap, t_capacity=0, line_graph_cutoff=None, atom_graph_cutoff=6.0,
                                     candidate_cutoff=8.0, padding=PaddingRule("far_self_loops"), device=device)


@pytest.mark.gpu
@pytest.mark.parametrize("n_cells,channels,hoist,fused,geometry", [
    (3, 128, None, True, "cubic"), (3, 64, None, True, "cubic"), (3, 256, None, True, "cubic"),
    ((6, 6, 6), 128, None, True, "cubic"), (3, 64, 0, True, "cubic"), (3, 128, 0, True, "cubic"),
    (3, 256, 0, True, "cubic"), ((6, 6, 6), 128, 10 ** 9, True, "cubic"), (3, 64, None, False, "cubic"),
    (3, 128, None, False, "cubic"), (3, 256, None, False, "cubic"), ((6, 6, 6), 128, None, False, "cubic"),
    ((10, 10, 10), 128, None, False, "cubic"),
    (3, 128, None, False, "triclinic_rotated"), ((6, 6, 6), 128, None, False, "triclinic_rotated"),
    ((6, 6, 6), 128, 0, False, "triclinic_rotated"), ((6, 6, 6), 64, 10 ** 9, False, "cubic"),
    ((10, 10, 20), 128, None, False, "cubic"), ((10, 10, 20), 128, 0, False, "cubic"),
    ((15, 15, 15), 128, None, False, "cubic")])
def test_mace_like_gpu_matches_oracle(device, n_cells, channels, hoist, fused, geometry, monkeypatch):
    """Energies within 1e-5 eV/atom and forces within 1e-4 eV/A of the FP64 oracle, through the
    fixed-capacity builder (padding rows present), bitwise reproducible. ``hoist`` None runs the
    node-factored pre-activation (P, Q per atom, the radial term per row, no edge GEMM); a number
    runs the edge GEMM form, with the receiver block formed per atom from that edge-list size
    (0: always, 10**9: never), so every evaluation order of z is checked; ``fused`` selects the
    fused node kernels or the unfused chain of GEMMs and contraction kernels; at 5 000 atoms the
    unfused node GEMMs take their split-plane grouped form. ``triclinic_rotated`` puts the crystal
    in a sheared cell rotated as a whole (no cell axis along x, y or z); 10 x 10 x 20 cells is the
    10 000-atom headline system, 15 x 15 x 15 cells (16 875 atoms) a system above it."""
    from fastmd_amd.engine.energy_derivative import EnergyDerivative
    from fastmd_amd.models import mace_like
    from fastmd_amd.models.mace_like import MaceLikeAdapter

    monkeypatch.setattr(mace_like, "FACTORED_Z", hoist is None)
    if hoist is not None:
        monkeypatch.setattr(mace_like, "HOIST_MIN_ROWS", hoist)
    monkeypatch.setattr(mace_like, "FUSED_NODE", fused)
    print(f"[mace] cells={n_cells} C={channels} hoist={hoist} fused={fused} {geometry}", flush=True)
    s = systems.perovskite(n_cells, sigma=0.2)  # displaced from the symmetric sites: sizeable forces
    if geometry == "triclinic_rotated":
        s = _triclinic_rotated(s)
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
    # the message kernels visit the atoms in the builder's spatial order: any order of the atoms
    # (here none, the index order) gives the same bits
    assert not torch.equal(builder.atom_order, torch.arange(n, dtype=torch.int32, device=device))
    saved_order = builder.batch.atom_order
    builder.batch.atom_order = None
    try:
        out3 = deriv(builder.batch, inputs, n_real=n)
    finally:
        builder.batch.atom_order = saved_order
    assert torch.equal(out3["e"], out["e"]) and torch.equal(out3["f"][0], out["f"][0])


@pytest.mark.gpu
@pytest.mark.parametrize("n,C", [(135, 128), (1080, 64), (37, 256)])
def test_mix_symcon_kernels(device, n, C):
    """fmd_mace_mix_symcon_f32 and its VJP half (small systems' node side, one launch each): P0 =
    A0 Wm0 and P1 = A1 Wm1 within fp32 of float64, the contraction B0, B1 the standalone kernel's on
    those P to fp32 rounding; gP0, gP1 the contraction VJP kernel's on float64 gB0 = g0 Wo0^T and
    gB1 = g1 Wo1^T (rounded to float32), with and without the vector gradient, with K = C and with
    the readout width 16 (the merged last layer); a ragged last tile of atoms (n % 16 != 0)."""
    from fastmd_amd import _abi
    from fastmd_amd.models.mace_like import MaceLike, MaceLikeConfig

    m = MaceLike(MaceLikeConfig(channels=C)).to(device)
    layer = m.layers[1]
    g = torch.Generator().manual_seed(5)
    d = lambda t: t.to(device).contiguous()  # noqa: E731
    A0, A1 = torch.randn(n, C, generator=g), torch.randn(n, 3, C, generator=g)
    elem = torch.randint(0, 3, (n,), generator=g, dtype=torch.int32)
    wm0t, wm1t = layer.Wm0.t().contiguous(), layer.Wm1.t().contiguous()
    P0, P1, B0, B1 = (torch.empty(n, C, device=device), torch.empty(n, 3, C, device=device),
                      torch.empty(n, C, device=device), torch.empty(n, 3, C, device=device))
    A0d, A1d, elemd = d(A0), d(A1), d(elem)  # (held: the kernels read them after the call returns)
    _abi.call("fmd_mace_mix_symcon_f32", A0d.data_ptr(), A1d.data_ptr(), wm0t.data_ptr(), wm1t.data_ptr(),
              elemd.data_ptr(), layer.Wc.data_ptr(), layer.Wd.data_ptr(), n, C, P0.data_ptr(), P1.data_ptr(),
              B0.data_ptr(), B1.data_ptr(), torch.cuda.current_stream().cuda_stream)
    r0 = A0.double() @ layer.Wm0.cpu().double()
    r1 = A1.double() @ layer.Wm1.cpu().double()
    rel = lambda x, r: float((x.cpu().double() - r).abs().max() / r.abs().max())  # noqa: E731
    assert rel(P0, r0) < 1e-5 and rel(P1, r1) < 1e-5
    B0s, B1s = torch.empty_like(B0), torch.empty_like(B1)
    _abi.call("fmd_mace_symcon_f32", P0.data_ptr(), P1.data_ptr(), elemd.data_ptr(), layer.Wc.data_ptr(),
              layer.Wd.data_ptr(), n, C, B0s.data_ptr(), B1s.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rel(B0, B0s.cpu().double()) < 1e-6 and rel(B1, B1s.cpu().double()) < 1e-6
    # VJP half
    for k0, with_vec in ((C, True), (C, False), (16, False)):
        g0 = torch.randn(n, k0, generator=g)
        wb0 = torch.randn(C, k0, generator=g) / k0 ** 0.5
        g1 = torch.randn(n, 3, C, generator=g) if with_vec else None
        gP0, gP1 = torch.empty(n, C, device=device), torch.empty(n, 3, C, device=device)
        g0d, wb0d, g1d = d(g0), d(wb0), (d(g1) if with_vec else None)
        _abi.call("fmd_mace_mix_symcon_bwd_f32", g0d.data_ptr(), k0, wb0d.data_ptr(), _abi.ptr(g1d),
                  layer.Wo1.data_ptr(), P0.data_ptr(), P1.data_ptr(), elemd.data_ptr(), layer.Wc.data_ptr(),
                  layer.Wd.data_ptr(), n, C, gP0.data_ptr(), gP1.data_ptr(), torch.cuda.current_stream().cuda_stream)
        gB0 = d((g0.double() @ wb0.double().t()).float())
        gB1 = d((g1.double() @ layer.Wo1.cpu().double().t()).float()) if with_vec else None
        rP0, rP1 = torch.empty_like(gP0), torch.empty_like(gP1)
        _abi.call("fmd_mace_symcon_bwd_f32", P0.data_ptr(), P1.data_ptr(), elemd.data_ptr(), layer.Wc.data_ptr(),
                  layer.Wd.data_ptr(), gB0.data_ptr(), _abi.ptr(gB1), n, C, rP0.data_ptr(), rP1.data_ptr(),
                  torch.cuda.current_stream().cuda_stream)
        assert rel(gP0, rP0.cpu().double()) < 1e-5 and rel(gP1, rP1.cpu().double()) < 1e-5


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
