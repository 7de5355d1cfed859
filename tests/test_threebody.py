"""Three-body Fourier angle basis: the oracle pinned by closed forms, symmetry and independent
derivatives (CPU); the HIP kernels (general rows and line-graph layout) against the float64
oracle with the reference's own tolerances (GPU,
fastmd/models/matris/op/triton_threebody_fourier.py:301-360)."""
import math

import numpy as np
import pytest

from oracle import threebody as otb
from fastmd_amd import systems
from fastmd_amd.adapters.protocol import PaddingRule

REF_FREQS = np.array([0.833447, 1.5861181, 2.5042067], np.float32)  # the reference's self-check frequencies
SCALE = math.sqrt(math.pi)  # FourierExpansion's scale (basis_function.py:120)


def _rand_unit(rng, n):
    v = rng.normal(size=(n, 3))
    return v / np.linalg.norm(v, axis=1, keepdims=True)


def _rotation(rng):
    q, r = np.linalg.qr(rng.normal(size=(3, 3)))
    return q * np.sign(np.diag(r))


# ----------------------------------------------------------------------------------- CPU


def test_oracle_closed_forms():
    """Orthogonal bonds: c = 0, theta = pi/2 exactly; 60 degrees: theta = acos(0.5 (1 - 1e-6));
    parallel / antiparallel: theta = acos(+-(1 - 1e-6)), the clamp that keeps acos' finite."""
    f = np.arange(1, 6, dtype=np.float64)  # FourierExpansion's default max_f = 5
    u = np.array([[1.0, 0, 0], [0, 1.0, 0], [0.5, math.sqrt(3) / 2, 0], [-1.0, 0, 0]])
    out = otb.fourier_basis(u, [0, 0, 0, 0], [1, 2, 0, 3], f, SCALE)
    assert out.shape == (4, 11)
    expect_t = [math.pi / 2, math.acos(0.5 * (1 - 1e-6)), math.acos(1 - 1e-6), math.acos(-(1 - 1e-6))]
    for row, t in zip(out, expect_t):
        assert abs(row[0] - 1 / math.sqrt(2) / SCALE) < 1e-15
        for k in range(5):
            assert abs(row[1 + k] - math.sin(t * (k + 1)) / SCALE) < 1e-12
            assert abs(row[6 + k] - math.cos(t * (k + 1)) / SCALE) < 1e-12
    # pi/2: sin(k pi/2) = 1, 0, -1, 0, 1; cos = 0, -1, 0, 1, 0
    assert np.allclose(out[0, 1:6] * SCALE, [1, 0, -1, 0, 1], atol=1e-12)
    assert np.allclose(out[0, 6:] * SCALE, [0, -1, 0, 1, 0], atol=1e-12)
    # the basis rows have the constant norm sqrt(1/2 + F) / scale
    assert np.allclose(np.linalg.norm(out, axis=1), math.sqrt(0.5 + 5) / SCALE)


def test_oracle_rotation_invariance_and_symmetry():
    rng = np.random.default_rng(7)
    u = _rand_unit(rng, 64)
    t = rng.integers(0, 64, 500)
    s = rng.integers(0, 64, 500)
    out = otb.fourier_basis(u, t, s, REF_FREQS, SCALE)
    assert np.allclose(otb.fourier_basis(u @ _rotation(rng).T, t, s, REF_FREQS, SCALE), out, atol=1e-12)
    assert np.array_equal(otb.fourier_basis(u, s, t, REF_FREQS, SCALE), out)  # the angle is symmetric
    g = rng.normal(size=out.shape)
    assert np.allclose(otb.fourier_basis_vjp(g, u, s, t, REF_FREQS, SCALE),
                       otb.fourier_basis_vjp(g, u, t, s, REF_FREQS, SCALE), atol=1e-12)


def test_oracle_vjp_against_finite_differences_and_autograd():
    """The explicit VJP against central differences of the forward (well-conditioned angles,
    vectors not normalised: the op differentiates the dot product as given) and against
    torch's float64 autograd of an independently written composition."""
    import torch

    rng = np.random.default_rng(11)
    u = _rand_unit(rng, 20) * rng.uniform(0.5, 1.0, (20, 1))
    t = rng.integers(0, 20, 60)
    s = (t + rng.integers(1, 20, 60)) % 20
    f = np.arange(1, 4, dtype=np.float64)
    g = rng.normal(size=(60, 7))
    gu = otb.fourier_basis_vjp(g, u, t, s, f, SCALE)
    h = 1e-6
    fd = np.zeros_like(u)
    for i in range(20):
        for x in range(3):
            up, um = u.copy(), u.copy()
            up[i, x] += h
            um[i, x] -= h
            fd[i, x] = ((otb.fourier_basis(up, t, s, f, SCALE) - otb.fourier_basis(um, t, s, f, SCALE)) * g).sum() / (2 * h)
    assert np.abs(gu - fd).max() < 1e-6 * max(1.0, np.abs(fd).max())

    ut = torch.tensor(u, dtype=torch.float64, requires_grad=True)
    cosang = torch.einsum("ij,ij->i", ut[torch.tensor(t)], ut[torch.tensor(s)]) * (1 - 1e-6)
    ang = torch.arccos(cosang)
    phase = ang[:, None] * torch.tensor(f)[None, :]
    basis = torch.cat([torch.full_like(ang[:, None], 2 ** -0.5), phase.sin(), phase.cos()], 1) / SCALE
    (basis * torch.tensor(g)).sum().backward()
    assert np.abs(ut.grad.numpy() - gu).max() < 1e-12 * max(1.0, np.abs(gu).max())
    assert np.abs(basis.detach().numpy() - otb.fourier_basis(u, t, s, f, SCALE)).max() < 1e-14


def test_oracle_vjp_linear_in_gout():
    rng = np.random.default_rng(3)
    u = _rand_unit(rng, 30)
    t, s = rng.integers(0, 30, 100), rng.integers(0, 30, 100)
    g1, g2 = rng.normal(size=(100, 7)), rng.normal(size=(100, 7))
    f = np.arange(1, 4, dtype=np.float64)
    a = otb.fourier_basis_vjp(2.0 * g1 - 3.0 * g2, u, t, s, f, SCALE)
    b = 2.0 * otb.fourier_basis_vjp(g1, u, t, s, f, SCALE) - 3.0 * otb.fourier_basis_vjp(g2, u, t, s, f, SCALE)
    assert np.allclose(a, b, atol=1e-10)
    # the constant column carries no gradient
    g3 = np.zeros((100, 7))
    g3[:, 0] = 1.0
    assert np.abs(otb.fourier_basis_vjp(g3, u, t, s, f, SCALE)).max() == 0.0


def test_ops_refuse_cpu_tensors():
    import torch

    from fastmd_amd.ops.threebody import threebody_fourier_basis

    u = torch.zeros(4, 3)
    i = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(ValueError, match="GPU tensor"):
        threebody_fourier_basis(u, i, i, torch.tensor(REF_FREQS), SCALE)


# ----------------------------------------------------------------------------------- GPU


def _eager(u, t, s, freqs, scale):
    """torch FP32 composition, the reference's eager baseline (:313-323)."""
    import torch

    ei = torch.index_select(u, 0, t)
    ej = torch.index_select(u, 0, s)
    ang = torch.acos(torch.sum(ei * ej, dim=1) * (1 - 1e-6))
    ph = torch.outer(ang, freqs.to(ang.dtype))
    return torch.cat([torch.full_like(ang[:, None], 2 ** -0.5), ph.sin(), ph.cos()], 1) / scale


def _errors(u, t, s, g, freqs, scale, fn):
    """(fwd max abs error, bwd max abs error / max |grad|) of fn and of the FP32 eager form,
    both against the float64 oracle."""
    import torch

    un, tn, sn, gn = u.cpu().numpy(), t.cpu().numpy(), s.cpu().numpy(), g.cpu().numpy()
    out64 = otb.fourier_basis(un, tn, sn, freqs.cpu().numpy(), scale)
    grad64 = otb.fourier_basis_vjp(gn, un, tn, sn, freqs.cpu().numpy(), scale)
    res = {}
    for name, f in (("eager", lambda x: _eager(x, t, s, freqs, scale)), ("hip", fn)):
        x = u.detach().clone().requires_grad_(True)
        out = f(x)
        out.backward(g)
        torch.cuda.synchronize()
        res[name] = (np.abs(out.detach().double().cpu().numpy() - out64).max(),
                     np.abs(x.grad.double().cpu().numpy() - grad64).max() / np.abs(grad64).max())
    return res


@pytest.mark.gpu
@pytest.mark.parametrize("rows,vectors", [(1024, 256), (152446, 26174)])
@pytest.mark.parametrize("nf", [3, 5])
def test_fourier_basis_matches_fp64(device, rows, vectors, nf):
    """The reference's own acceptance (:342-360): within 2x / 4x the FP32 eager error of FP64
    (plus 1e-6 / 1e-5) on all pairs, FP32 tolerance (5e-6 / 1e-5) on |t| < 0.99."""
    import torch

    from fastmd_amd.ops.threebody import threebody_fourier_basis

    print(f"[fourier] rows={rows} vectors={vectors} nf={nf}", flush=True)
    gen = torch.Generator().manual_seed(rows + nf)
    freqs = (torch.tensor(REF_FREQS) if nf == 3 else torch.arange(1, nf + 1, dtype=torch.float32)).to(device)
    unit = torch.nn.functional.normalize(torch.randn(vectors, 3, generator=gen), dim=1).to(device)
    target = torch.randint(0, vectors, (rows,), generator=gen).to(device)
    source = torch.randint(0, vectors, (rows,), generator=gen).to(device)
    source = torch.where(source == target, (source + 1) % vectors, source)
    grad = torch.randn(rows, 1 + 2 * nf, generator=gen).to(device)

    def hip(x, t=target, s=source):
        return threebody_fourier_basis(x, t, s, freqs, SCALE, check_range=True)

    err = _errors(unit, target, source, grad, freqs, SCALE, hip)
    assert err["hip"][0] <= 2 * err["eager"][0] + 1e-6, err
    assert err["hip"][1] <= 4 * err["eager"][1] + 1e-5, err
    well = (unit[target] * unit[source]).sum(1).abs() < 0.99
    tw, sw = target[well], source[well]
    err_w = _errors(unit, tw, sw, grad[well], freqs, SCALE, lambda x: hip(x, tw, sw))
    assert err_w["hip"][0] < 5e-6 and err_w["hip"][1] < 1e-5, err_w


@pytest.mark.gpu
def test_fourier_basis_deterministic_and_empty(device):
    import torch

    from fastmd_amd.ops.threebody import fourier_basis_vjp, threebody_fourier_basis

    gen = torch.Generator().manual_seed(5)
    freqs = torch.tensor(REF_FREQS, device=device)
    unit = torch.nn.functional.normalize(torch.randn(3000, 3, generator=gen), dim=1).to(device)
    t = torch.randint(0, 3000, (50000,), generator=gen).to(device)
    s = torch.randint(0, 3000, (50000,), generator=gen).to(device)
    g = torch.randn(50000, 7, generator=gen).to(device)
    a = fourier_basis_vjp(g, unit, t, s, freqs, SCALE)
    b = fourier_basis_vjp(g, unit, t, s, freqs, SCALE)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # int32 and int64 indices agree bit for bit
    assert torch.equal(threebody_fourier_basis(unit, t, s, freqs, SCALE),
                       threebody_fourier_basis(unit, t.int(), s.int(), freqs, SCALE))
    x = unit.clone().requires_grad_(True)
    e = torch.zeros(0, dtype=torch.int64, device=device)
    out = threebody_fourier_basis(x, e, e, freqs, SCALE)
    assert out.shape == (0, 7)
    out.sum().backward()
    assert x.grad.shape == (3000, 3) and not x.grad.any()
    with pytest.raises(IndexError):
        threebody_fourier_basis(unit, t, s + 3000, freqs, SCALE, check_range=True)


def _line(device, n_atoms, line_cutoff, t_cap=None, u_cap=None):
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    s = systems.perovskite_atoms(n_atoms)
    u_cap = int(round(15.3 * n_atoms / 2)) + 64 if u_cap is None else u_cap
    t_cap = 40 * n_atoms if t_cap is None else t_cap
    builder = FixedCapacityGraphBuilder(cell=torch.tensor(s.cell, dtype=torch.float32),
                                        atomic_numbers=torch.ones(n_atoms), u_capacity=u_cap, t_capacity=t_cap,
                                        atom_graph_cutoff=6.0, line_graph_cutoff=line_cutoff, candidate_cutoff=8.0,
                                        padding=PaddingRule("far_self_loops"), device=device)
    builder.build(torch.tensor(s.positions, dtype=torch.float64, device=device))
    return builder


@pytest.mark.gpu
@pytest.mark.parametrize("n_atoms,line_cutoff", [(135, 3.5), (1080, 3.0), (5000, 3.0), (5000, 3.5)])
def test_fourier_line_matches_rows_and_fp64(device, n_atoms, line_cutoff):
    """The line-graph kernels against the general ones on the line graph's own triplet rows:
    forward bit-exact over every row (real and padding); VJP (padding gout zero) against the
    deterministic general VJP and the float64 oracle; repeated runs bitwise equal; accumulate
    adds onto what the rows held."""
    import torch

    from fastmd_amd.ops.threebody import (LineGraph, fourier_basis_vjp, fourier_line_vjp, threebody_fourier_basis,
                                          threebody_fourier_line)

    print(f"[fourier line] n_atoms={n_atoms} cutoff={line_cutoff}", flush=True)
    b = _line(device, n_atoms, line_cutoff)
    assert not bool(b._overflow.item())
    lg = LineGraph.from_builder(b)
    t_real = int(b.pair_offsets[-1].item())
    assert 0 < t_real <= lg.t_cap
    gen = torch.Generator().manual_seed(n_atoms)
    freqs = torch.tensor(REF_FREQS, device=device)
    unit = torch.nn.functional.normalize(torch.randn(b.e_capacity, 3, generator=gen), dim=1).to(device)
    tgt, src = b.line_graph[:, 2], b.line_graph[:, 4]
    out = threebody_fourier_line(unit, lg, freqs, SCALE)
    ref = threebody_fourier_basis(unit, tgt, src, freqs, SCALE)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)

    g = torch.randn(lg.t_cap, 7, generator=gen).to(device)
    g[t_real:] = 0
    x = unit.clone().requires_grad_(True)
    threebody_fourier_line(x, lg, freqs, SCALE).backward(g)
    general = fourier_basis_vjp(g, unit, tgt, src, freqs, SCALE)
    again = torch.zeros_like(unit)
    fourier_line_vjp(g, unit, lg, freqs, SCALE, out=again, accumulate=False)
    torch.cuda.synchronize()
    assert torch.equal(x.grad, again)
    scale = general.abs().max()
    assert (x.grad - general).abs().max() <= 1e-6 * scale
    tn, sn = tgt[:t_real].cpu().numpy(), src[:t_real].cpu().numpy()
    g64 = otb.fourier_basis_vjp(g[:t_real].cpu().numpy(), unit.cpu().numpy(), tn, sn, REF_FREQS, SCALE)
    x32 = unit.clone().requires_grad_(True)
    _eager(x32, tgt[:t_real].long(), src[:t_real].long(), freqs, SCALE).backward(g[:t_real])
    torch.cuda.synchronize()
    err_eager = np.abs(x32.grad.double().cpu().numpy() - g64).max() / np.abs(g64).max()
    err_line = np.abs(x.grad.double().cpu().numpy() - g64).max() / np.abs(g64).max()
    assert err_line <= 4 * err_eager + 1e-5, (err_line, err_eager)  # the reference's bound (:358)
    # rows that are not short bonds get no gradient
    short = b.short_flags.bool()
    assert not x.grad[~short].any()
    # accumulate onto a non-zero buffer: short rows = old + grad, others unchanged
    base = torch.randn(b.e_capacity, 4, generator=gen).to(device)
    acc = base.clone()
    fourier_line_vjp(g, unit, lg, freqs, SCALE, out=acc, accumulate=True)
    torch.cuda.synchronize()
    assert torch.equal(acc[:, 3], base[:, 3]) and torch.equal(acc[~short], base[~short])
    assert torch.equal(acc[short, :3], base[short, :3] + x.grad[short])


@pytest.mark.gpu
def test_fourier_line_overflow_topology(device):
    """An overflowed build (edges above the capacity) carries the all-loop triplet topology: the
    line forward still equals the general one on every row, and the VJP stays in bounds."""
    import torch

    from fastmd_amd.ops.threebody import LineGraph, threebody_fourier_basis, threebody_fourier_line

    b = _line(device, 135, 3.5, u_cap=300)
    assert bool(b._overflow.item())
    lg = LineGraph.from_builder(b)
    freqs = torch.arange(1, 4, dtype=torch.float32, device=device)
    gen = torch.Generator().manual_seed(1)
    unit = torch.nn.functional.normalize(torch.randn(b.e_capacity, 3, generator=gen), dim=1).to(device)
    x = unit.clone().requires_grad_(True)
    out = threebody_fourier_line(x, lg, freqs, SCALE)
    ref = threebody_fourier_basis(unit, b.line_graph[:, 2], b.line_graph[:, 4], freqs, SCALE)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    out.sum().backward()
    torch.cuda.synchronize()
    assert not x.grad.any()  # every row is padding


@pytest.mark.gpu
@pytest.mark.parametrize("n_atoms", [135, 5000])
def test_angle_bond_atom_segment_sums(device, n_atoms):
    """The line graph's CSR layouts drive the deterministic segment sums of a three-body layer:
    angles -> their first bond (edge_triplet_offsets over the directed rows, identity rows) and
    bonds -> atoms (short_offsets over bond_rows); each against float64 sums grouped by the
    triplet rows' own bond and atom columns."""
    import torch

    from fastmd_amd.ops.csr_segment_sum import Csr, segment_sum_csr

    print(f"[angle sums] n_atoms={n_atoms}", flush=True)
    b = _line(device, n_atoms, 3.5)
    t_real = int(b.pair_offsets[-1].item())
    gen = torch.Generator().manual_seed(2)
    vals = torch.randn(b.t_capacity, 64, generator=gen).to(device)
    bond = segment_sum_csr([(vals, Csr(b.edge_triplet_offsets, None, b.t_capacity), 0, 1.0, None)],
                           b.e_capacity, 64)
    atom = segment_sum_csr([(bond, Csr(b.short_offsets, b.bond_rows), 0, 1.0, None)], n_atoms, 64)
    torch.cuda.synchronize()
    line = b.line_graph[:t_real].cpu().numpy().astype(np.int64)
    v64 = vals[:t_real].double().cpu().numpy()
    want_bond = np.zeros((b.e_capacity, 64))
    np.add.at(want_bond, line[:, 2], v64)
    want_atom = np.zeros((n_atoms, 64))
    np.add.at(want_atom, line[:, 0], v64)
    assert np.abs(bond.double().cpu().numpy() - want_bond).max() < 1e-4
    assert np.abs(atom.double().cpu().numpy() - want_atom).max() < 1e-3
