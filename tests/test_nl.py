"""(a) Neighbour list: the oracle pinned against the reference's own checks (CPU), and the HIP
builder bit-exact against the oracle (GPU)."""
import math

import numpy as np
import pytest

from oracle import nl as onl
from fastmd_amd import systems
from fastmd_amd.adapters.protocol import PaddingRule

F32 = np.float32


def _crystal():
    """Perturbed 3x3x3 simple-cubic crystal in a slightly triclinic cell
    (tests/test_fixed_capacity_boundary.py:43-53 of the reference, seed 1234)."""
    rng = np.random.default_rng(1234)
    cell = np.array([[6.0, 0.0, 0.0], [0.3, 6.1, 0.0], [0.2, -0.25, 5.9]])
    grid = np.stack(np.meshgrid(*(np.arange(3),) * 3, indexing="ij"), -1).reshape(-1, 3)
    frac = (grid + 0.5 + rng.uniform(-0.08, 0.08, grid.shape)) / 3.0
    return cell, frac @ cell


def _lattice(n_side, spacing, jitter, seed):
    """tests/test_ragged_builder_overflow.py:33-43 of the reference (positions float32)."""
    rng = np.random.default_rng(seed)
    grid = np.stack(np.meshgrid(*(np.arange(n_side),) * 3, indexing="ij"), -1)
    positions = (grid.reshape(-1, 3) + 0.5) * spacing
    positions = positions + rng.uniform(-jitter, jitter, positions.shape)
    return np.eye(3) * n_side * spacing, positions.astype(np.float32).astype(np.float64)


def _inv32(cell):
    """The builders' inverse: of the float32-rounded cell, in float64, rounded to float32."""
    return np.linalg.inv(np.asarray(cell, dtype=F32).astype(np.float64)).astype(F32)


def _oracle_build(cell, positions, cutoff, skin, e_cap, pad=None, ref_positions=None, inv=None,
                  minimum_image=False):
    cell32 = cell.astype(F32)
    inv = _inv32(cell) if inv is None else inv
    ref = positions if ref_positions is None else ref_positions
    _, wraps, wrapped = onl.wrap(ref, inv, cell32)
    bmax = onl.estimate_max_neighbors(cutoff + skin, safety_factor=2.0)
    cand = onl.candidates(wrapped, cell32, F32((cutoff + skin) ** 2), bmax)
    if pad is None:
        pad, _ = onl.self_loop_image(cell, cutoff)
    b = onl.build(positions, inv, cell32, cand, np.asarray(ref, dtype=F32), wraps, F32(cutoff * cutoff),
                  F32(skin + 1e-6), pad, e_cap, minimum_image=minimum_image)
    return cand, b, wrapped


# ------------------------------------------------------------------------------- CPU: oracle pins
def test_estimate_max_neighbors_known_answers():
    # tests/test_ragged_builder_overflow.py:328-336 of the reference
    for cutoff, expected in ((6.0 + 1e-6, 640), (5.0, 368), (3.0, 80), (0.0, 0)):
        assert onl.estimate_max_neighbors(cutoff=cutoff, safety_factor=2.0) == expected
    from fastmd_amd.graph.neighbor_list_backend import estimate_max_neighbors

    for cutoff in np.linspace(0.5, 12.0, 50):
        assert estimate_max_neighbors(float(cutoff), safety_factor=2.0) == onl.estimate_max_neighbors(
            float(cutoff), safety_factor=2.0)
    assert onl.estimate_max_neighbors(8.0, safety_factor=2.0) == 1504


def test_growth_rule():
    from fastmd_amd.graph.gpu_graph_builder import grown_max_neighbors

    for cap, mx in ((8, 9), (8, 100), (80, 81), (16, 17), (1, 1)):
        assert grown_max_neighbors(cap, mx) == max(2 * cap, math.ceil(mx / 16) * 16) == onl.grown_max_neighbors(cap, mx)


@pytest.mark.parametrize("case", ["perovskite", "crystal", "lattice"])
def test_oracle_edges_equal_fp64_brute_force(case):
    """The oracle's real edges are the FP64 dense pair set, up to pairs within 1e-5 A of the
    cutoff (tests/test_fixed_capacity_boundary.py:358-365 of the reference)."""
    if case == "perovskite":
        s = systems.perovskite(3)
        cell, pos, cutoff = s.cell, s.positions, 6.0
    elif case == "crystal":
        cell, pos = _crystal()
        cutoff = 3.0
    else:
        cell, pos = _lattice(5, 1.6, 0.15, 0)
        cutoff = 3.0
    cand, b, wrapped = _oracle_build(cell, pos, cutoff, 1.0, 100000)
    e = b.n_edges
    got = {(int(c), int(n), *map(int, i)): float(d) for c, n, i, d in
           zip(b.center[:e], b.neighbor[:e], b.images[:e], b.distances[:e])}
    dense = onl.dense_pairs(wrapped, cell.astype(F32), cutoff)
    near = {k for k, d in dense.items() if abs(d - cutoff) < 1e-5} | {k for k, d in got.items() if abs(d - cutoff) < 1e-5}
    assert set(got) - near == set(dense) - near
    assert onl.canonical_order_ok(b.center[:e], b.neighbor[:e], b.images[:e], pos.shape[0])
    for k, d in got.items():  # distances are the rows' own
        assert abs(d - dense.get(k, d)) < 1e-4


def test_perovskite_edge_statistics():
    """15.21 edges/atom at a = 6.2, rc = 6 (E = 2 054 at 135 atoms), 50 candidates at 8 A."""
    s = systems.perovskite(3)
    cand, b, _ = _oracle_build(s.cell, s.positions, 6.0, 2.0, 2176)
    assert b.n_edges == 2054 and not b.overflow and b.isolated == 0
    assert cand.num_neighbors.max() == 52 and cand.capacity_valid


def test_padding_layout_and_overflow_flag():
    s = systems.perovskite(3)
    cell = s.cell
    image, length = onl.self_loop_image(cell, 6.0)
    assert image == (1, 0, 0) and length == pytest.approx(18.6)  # m = 1: |a| = 18.6 >= 2 rc
    _, b, _ = _oracle_build(cell, s.positions, 6.0, 2.0, 2176)
    rows = np.arange(b.n_edges, 2176)
    assert np.array_equal(b.center[rows], (rows - b.n_edges) % 135)  # round robin
    assert np.array_equal(b.neighbor[rows], b.center[rows])
    assert (b.images[rows] == np.array(image)).all()
    _, small, _ = _oracle_build(cell, s.positions, 6.0, 2.0, 1000)
    assert small.overflow and small.n_edges == 2054
    assert onl.fixed_capacity_exceeded(2054, False, 1000)


def test_fixed_capacity_truth_table():
    # tests/test_fixed_capacity_boundary.py:111-120 of the reference (edges only)
    for edges, invalid, expected in ((31, False, False), (32, False, False), (33, False, True),
                                     (34, False, True), (30, True, True)):
        assert onl.fixed_capacity_exceeded(edges, invalid, 32) == expected


def test_padding_rule_validation_table():
    # tests/test_fixed_capacity_boundary.py:121-129 of the reference
    from fastmd_amd.adapters.protocol import PaddingRule

    for kwargs, message in (({"kind": "zero_loops"}, "unknown kind"), ({"min_length": -1.0}, "min_length"),
                            ({"min_length": float("nan")}, "min_length"),
                            ({"kind": "sink_atoms", "min_length": 1.0}, "far_self_loops only"),
                            ({"kind": "far_self_loops", "pad_vector": (1.0, 0.0, 0.0)}, "exact_rc_loops only"),
                            ({"kind": "exact_rc_loops", "pad_vector": (1.0, 0.0)}, "three finite"),
                            ({"placement": "one_row"}, "unknown placement")):
        with pytest.raises(ValueError, match=message):
            PaddingRule(**kwargs)


def test_reused_candidates_equal_fresh_build():
    """A build over reused candidates equals a fresh build bitwise after moves within the skin
    (tests/test_fixed_capacity_boundary.py:439-461 of the reference), across wrap changes."""
    s = systems.perovskite(3)
    rng = np.random.default_rng(5)
    moved = s.positions + rng.normal(0, 0.2, s.positions.shape)
    moved[:, 0] -= s.positions[:, 0].min() + 0.05  # atoms of the x = 0 face leave the cell: wraps change
    earlier = moved - rng.normal(0, 0.1, moved.shape)  # the refresh's positions, within the skin
    _, reused, _ = _oracle_build(s.cell, moved, 6.0, 2.0, 2400, ref_positions=earlier)
    _, fresh, _ = _oracle_build(s.cell, moved, 6.0, 2.0, 2400)
    assert reused.candidate_valid and not reused.overflow
    assert (reused.wrap_delta != 0).any()
    e = fresh.n_edges
    assert reused.n_edges == e
    for a, b in ((reused.center, fresh.center), (reused.neighbor, fresh.neighbor), (reused.images, fresh.images)):
        assert np.array_equal(a[:e], b[:e])
    # a lattice jump of the unwrapped coordinate is motion for this builder: the skin test fails
    jumped = moved.copy()
    jumped[:3] += s.cell[0]
    _, bad, _ = _oracle_build(s.cell, jumped, 6.0, 2.0, 2400, ref_positions=moved)
    assert not bad.candidate_valid and bad.overflow


def _edge_keys(b, wraps):
    """The build's rows as (centre, neighbour, image) in the frame of the caller's coordinates."""
    e = b.n_edges
    w = wraps.astype(np.int64)
    img = b.images[:e].astype(np.int64) - w[b.neighbor[:e]] + w[b.center[:e]]
    return {(int(i), int(j), *map(int, k)) for i, j, k in zip(b.center[:e], b.neighbor[:e], img)}


def test_minimum_image_build_ignores_lattice_jumps():
    """fixed_capacity_builder.py:2233-2245: with minimum_image, atoms the caller wrapped by lattice
    vectors since the refresh (ASE's atoms.wrap()) keep the skin test valid and give the FP64
    brute-force pair set of the unwrapped coordinates (rows within 1e-4 A of the cutoff aside),
    on a sheared cell; the jumps leave the wrap delta. Without it the skin test fails."""
    import md_oracle

    s = systems.perovskite(3)
    cell = s.cell + np.array([[0.0, 0.0, 0.0], [0.9, 0.0, 0.0], [0.4, -0.6, 0.0]])
    positions = (s.positions @ np.linalg.inv(s.cell)) @ cell
    rng = np.random.default_rng(11)
    moved = positions + rng.normal(0, 0.15, positions.shape)
    jumps = rng.integers(-2, 3, size=positions.shape)
    jumps[::3] = 0
    jumped = moved + jumps @ cell
    inv = _inv32(cell)
    cell32 = cell.astype(F32)
    _, plain, _ = _oracle_build(cell, moved, 6.0, 2.0, 4000, ref_positions=positions)
    _, mi, _ = _oracle_build(cell, jumped, 6.0, 2.0, 4000, ref_positions=positions, minimum_image=True)
    _, bad, _ = _oracle_build(cell, jumped, 6.0, 2.0, 4000, ref_positions=positions)
    assert plain.candidate_valid and mi.candidate_valid and not bad.candidate_valid and not mi.overflow
    assert abs(float(mi.max_displacement) - float(plain.max_displacement)) < 1e-4
    # the minimum-image wrap delta is the unjumped one's shifted by the wrap change minus the jump
    _, w_moved, _ = onl.wrap(moved, inv, cell32)
    _, w_jumped, _ = onl.wrap(jumped, inv, cell32)
    assert np.array_equal(mi.wrap_delta, plain.wrap_delta + (w_jumped - w_moved) - jumps)
    ours = _edge_keys(mi, w_jumped.astype(np.int64) - jumps)
    ii, jj, img = md_oracle.PairList(cell).pairs(moved)
    brute = {(int(i), int(j), *map(int, k)) for i, j, k in zip(ii, jj, img)}
    assert len(brute) > 1500
    vec = lambda t: moved[t[1]] + np.asarray(t[2:]) @ cell - moved[t[0]]  # noqa: E731
    assert all(abs(np.linalg.norm(vec(t)) - 6.0) < 1e-4 for t in ours ^ brute)


def test_morton_order_is_a_local_permutation():
    """The builder's atom order (fixed_capacity_builder.morton_order): a permutation of the rows, a
    union's systems one after the other, consecutive atoms close in space."""
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import morton_order

    frac = torch.rand(4000, 3, generator=torch.Generator().manual_seed(0))
    order = morton_order(frac)
    assert order.dtype == torch.int32 and sorted(order.tolist()) == list(range(4000))
    step = (frac[order[1:].long()] - frac[order[:-1].long()]).norm(dim=1).mean()
    assert float(step) < 0.25 * float((frac[1:] - frac[:-1]).norm(dim=1).mean())
    system = torch.repeat_interleave(torch.arange(4), 1000).to(torch.int32)
    order = morton_order(frac, system)
    assert torch.equal(system[order.long()], system)  # grouped by system, in system order


def test_window_fold():
    st = {"overflow": False, "capacity_overflow": False, "max_edges": 0, "max_isolated": 0}
    st = onl.window_fold(st, 10, False, False, 0, 32, True)
    st = onl.window_fold(st, 40, False, True, 2, 32, False)
    assert st == {"overflow": True, "capacity_overflow": True, "max_edges": 40, "max_isolated": 2}


# ------------------------------------------------------------------------------- GPU: HIP vs oracle
def _gpu_builder(cell, n, cutoff, skin, u_cap, device):
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    return FixedCapacityGraphBuilder(cell=torch.tensor(cell, dtype=torch.float32), atomic_numbers=torch.ones(n),
                                     u_capacity=u_cap, t_capacity=0, line_graph_cutoff=None, atom_graph_cutoff=cutoff,
                                     candidate_cutoff=cutoff + skin, padding=PaddingRule("far_self_loops"), device=device)


def _assert_build_equal(builder, ob, cand=None):
    n = builder.n_real
    e_cap = builder.e_capacity
    off = builder.edge_offsets.cpu().numpy()
    assert np.array_equal(off, ob.edge_offsets)
    assert np.array_equal(builder.edge_counts.cpu().numpy(), ob.edge_counts)
    ec = min(ob.n_edges, e_cap)
    assert np.array_equal(builder.center.cpu().numpy(), ob.center)
    assert np.array_equal(builder.neighbor.cpu().numpy(), ob.neighbor)
    assert np.array_equal(builder.images.cpu().numpy(), ob.images)
    assert np.array_equal(builder.distances.cpu().numpy()[:ec], ob.distances[:ec])
    assert np.array_equal(builder.frac_coords.cpu().numpy(), ob.frac)
    assert np.array_equal(builder.wrap_delta.cpu().numpy(), ob.wrap_delta)
    assert np.array_equal(builder.positions.cpu().numpy(), ob.wrapped)
    assert builder._max_displacement.cpu().numpy()[0] == ob.max_displacement
    assert bool(builder._candidate_valid.item()) == ob.candidate_valid
    assert bool(builder._overflow.item()) == ob.overflow
    assert int(builder._isolated_atom_count.item()) == ob.isolated
    ei = builder.batch.edge_index.cpu().numpy()
    assert np.array_equal(ei[:, 0], ob.center) and np.array_equal(ei[:, 1], ob.neighbor)
    assert np.array_equal(builder.batch.edge_image.cpu().numpy(), ob.images.astype(F32))
    rev = builder.edge_reverse.cpu().numpy()
    assert np.array_equal(rev, onl.reverse(ob.center, ob.neighbor, ob.images, ob.edge_offsets, e_cap))
    if cand is not None:
        assert np.array_equal(builder.num_neighbors.cpu().numpy(), cand.num_neighbors)
        assert np.array_equal(builder.neighbor_matrix.cpu().numpy(), cand.neighbor_matrix)
        assert np.array_equal(builder.neighbor_shifts.cpu().numpy(), cand.neighbor_shifts)


@pytest.mark.gpu
@pytest.mark.parametrize("n_atoms", [135, 1080, 3430, 10000, 16875, 40000])
def test_builder_bit_exact(device, n_atoms):
    """Candidates, rows, flags and published buffers bit-exact vs the oracle, on the fused
    single-workgroup path (<= 1024 atoms) and the multi-block path, fresh and with reused
    candidates after seeded moves (wraps change, skin still valid)."""
    import torch

    print(f"[nl] n_atoms={n_atoms}", flush=True)
    s = systems.perovskite_atoms(n_atoms)
    cutoff, skin = 6.0, 2.0
    u_cap = int(round(15.3 * n_atoms / 2)) + 64
    builder = _gpu_builder(s.cell, n_atoms, cutoff, skin, u_cap, device)
    pos = torch.tensor(s.positions, dtype=torch.float64, device=device)
    builder.build(pos, rebuild_candidates=True)
    inv = builder.inv_cell.cpu().numpy()
    cand, ob, _ = _oracle_build(s.cell, s.positions, cutoff, skin, builder.e_capacity, inv=inv)
    torch.cuda.synchronize()
    _assert_build_equal(builder, ob, cand)
    cell32 = s.cell.astype(F32)
    _, wraps, _ = onl.wrap(s.positions, inv, cell32)
    rng = np.random.default_rng(7)
    for sigma, jump, valid in ((0.08, False, True), (0.25, True, False)):
        moved = s.positions + rng.normal(0, sigma, s.positions.shape)
        if jump:
            moved[: n_atoms // 10] += s.cell[1]
        builder.build(torch.tensor(moved, device=device), rebuild_candidates=False)
        ob2 = onl.build(moved, inv, cell32, cand, s.positions.astype(F32), wraps, F32(36.0), F32(2.0 + 1e-6),
                        onl.self_loop_image(s.cell, cutoff)[0], builder.e_capacity)
        torch.cuda.synchronize()
        _assert_build_equal(builder, ob2)
        assert ob2.candidate_valid == valid


@pytest.mark.gpu
def test_builder_overflow_and_triclinic(device):
    """An edge count above e_cap sets the overflow flag and keeps every stored index in range;
    a triclinic crystal with a cutoff above half the cell (many images) stays bit-exact."""
    import torch

    s = systems.perovskite(3)
    builder = _gpu_builder(s.cell, 135, 6.0, 2.0, 500, device)
    builder.build(torch.tensor(s.positions, device=device))
    cand, ob, _ = _oracle_build(s.cell, s.positions, 6.0, 2.0, 1000, inv=builder.inv_cell.cpu().numpy())
    torch.cuda.synchronize()
    _assert_build_equal(builder, ob, cand)
    assert ob.overflow and bool(builder._overflow.item())
    cell, pos = _crystal()
    builder = _gpu_builder(cell, pos.shape[0], 3.0, 1.0, 1500, device)
    builder.build(torch.tensor(pos, device=device))
    cand, ob, _ = _oracle_build(cell, pos, 3.0, 1.0, 3000, inv=builder.inv_cell.cpu().numpy())
    torch.cuda.synchronize()
    _assert_build_equal(builder, ob, cand)


@pytest.mark.gpu
@pytest.mark.parametrize("n_atoms", [135, 3430])
def test_builder_minimum_image_bit_exact(device, n_atoms):
    """minimum_image builds bit-exact vs the oracle on the single-workgroup and the multi-block
    path, with atoms wrapped by lattice vectors since the refresh."""
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    print(f"[nl minimum image] n_atoms={n_atoms}", flush=True)
    s = systems.perovskite_atoms(n_atoms)
    builder = FixedCapacityGraphBuilder(cell=torch.tensor(s.cell, dtype=torch.float32),
                                        atomic_numbers=torch.ones(n_atoms), u_capacity=9 * n_atoms + 64, t_capacity=0,
                                        line_graph_cutoff=None, atom_graph_cutoff=6.0, candidate_cutoff=8.0,
                                        minimum_image=True, padding=PaddingRule("far_self_loops"), device=device)
    builder.build(torch.tensor(s.positions, dtype=torch.float64, device=device), rebuild_candidates=True)
    inv = builder.inv_cell.cpu().numpy()
    cell32 = s.cell.astype(F32)
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    cand = onl.candidates(wrapped, cell32, F32(64.0), builder.buffer_max)
    rng = np.random.default_rng(n_atoms)
    moved = s.positions + rng.normal(0, 0.15, s.positions.shape)
    jumps = rng.integers(-1, 2, size=s.positions.shape)
    jumps[::2] = 0
    jumped = moved + jumps @ s.cell
    builder.build(torch.tensor(jumped, device=device), rebuild_candidates=False)
    ob = onl.build(jumped, inv, cell32, cand, s.positions.astype(F32), wraps, F32(36.0), F32(2.0 + 1e-6),
                   onl.self_loop_image(s.cell, 6.0)[0], builder.e_capacity, minimum_image=True)
    torch.cuda.synchronize()
    _assert_build_equal(builder, ob)
    assert ob.candidate_valid and not ob.overflow


@pytest.mark.gpu
def test_shared_candidates_follow_the_owner(device):
    """candidates_from: a builder of a larger capacity reads (and refreshes) the owner's candidate
    list; its builds equal the owner's bitwise."""
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    s = systems.perovskite(6)
    n = s.n_atoms
    kw = dict(cell=torch.tensor(s.cell, dtype=torch.float32), atomic_numbers=torch.ones(n), atom_graph_cutoff=6.0,
              candidate_cutoff=8.0, t_capacity=0, line_graph_cutoff=None, padding=PaddingRule("far_self_loops"),
              device=device)
    owner = FixedCapacityGraphBuilder(u_capacity=9 * n, **kw)
    follower = FixedCapacityGraphBuilder(u_capacity=9 * n + 512, candidates_from=owner, **kw)
    assert follower.neighbor_matrix.data_ptr() == owner.neighbor_matrix.data_ptr()
    with pytest.raises(RuntimeError, match="refresh_candidates"):
        follower.build(torch.tensor(s.positions, device=device), rebuild_candidates=False)
    rng = np.random.default_rng(3)
    for step in range(3):
        q = torch.tensor(s.positions + rng.normal(0, 0.1, s.positions.shape), device=device)
        (owner if step == 0 else follower).build(q, rebuild_candidates=step != 1)
        owner.build(q, rebuild_candidates=False)
        follower.build(q, rebuild_candidates=False)
        e = int(owner.edge_offsets[-1])
        for name in ("edge_offsets", "frac_coords", "positions"):
            assert torch.equal(getattr(owner, name), getattr(follower, name)), name
        for name in ("center", "neighbor", "images", "distances"):
            assert torch.equal(getattr(owner, name)[:e], getattr(follower, name)[:e]), name
    with pytest.raises(ValueError, match="same system"):
        FixedCapacityGraphBuilder(u_capacity=9 * n, candidates_from=owner, **dict(kw, candidate_cutoff=7.0))


@pytest.mark.gpu
@pytest.mark.parametrize("spacing", [1.1, 1.0])
def test_truncated_candidate_rows_are_deterministic(device, spacing):
    """Rows with more candidates than slots (bmax 1 504 at 8 A): at 1.1 A spacing (~1 600 per atom)
    the row keeps the sorted first bmax, bit-exact vs the oracle; at 1.0 A (~2 140, more than the
    LDS key buffer of 2 048) it is stored empty. Either way repeated refreshes give the same rows,
    the counts are the oracle's, the capacity flag is cleared and the builder raises
    NeighborOverflowError."""
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder
    from fastmd_amd.graph.neighbor_list_backend import NeighborOverflowError

    side = 13 if spacing == 1.1 else 14
    grid = np.stack(np.meshgrid(*(np.arange(side),) * 3, indexing="ij"), -1).reshape(-1, 3)
    cell = np.eye(3) * side * spacing
    rng = np.random.default_rng(side)
    positions = (grid + 0.5) * spacing + rng.uniform(-0.02, 0.02, grid.shape)
    n = positions.shape[0]
    builder = FixedCapacityGraphBuilder(cell=torch.tensor(cell, dtype=torch.float32), atomic_numbers=torch.ones(n),
                                        u_capacity=64, t_capacity=0, line_graph_cutoff=None, atom_graph_cutoff=6.0,
                                        candidate_cutoff=8.0, padding=PaddingRule("far_self_loops"), device=device)
    bmax = builder.buffer_max
    pos = torch.tensor(positions, dtype=torch.float64, device=device)
    rows = []
    for _ in range(3):
        builder.refresh_candidates(pos)
        rows.append((builder.neighbor_matrix.clone(), builder.neighbor_shifts.clone(), builder.num_neighbors.clone()))
    for other in rows[1:]:
        assert all(torch.equal(a, b) for a, b in zip(rows[0], other))
    assert int(builder._candidate_capacity_valid.item()) == 0
    with pytest.raises(NeighborOverflowError):
        builder.assert_candidate_capacity()
    cell32 = cell.astype(F32)
    _, _, wrapped = onl.wrap(positions, builder.inv_cell.cpu().numpy(), cell32)
    cand = onl.candidates(wrapped, cell32, F32(64.0), bmax)
    num = rows[0][2].cpu().numpy()
    assert np.array_equal(num, cand.num_neighbors)
    nm = rows[0][0].cpu().numpy()
    fits = num <= 2048
    assert fits.all() if spacing == 1.1 else not fits.any()
    assert (num > bmax).all()
    assert np.array_equal(nm[fits], cand.neighbor_matrix[fits])
    assert np.array_equal(rows[0][1].cpu().numpy()[fits], cand.neighbor_shifts[fits])
    assert (nm[~fits] == n).all() and (rows[0][1].cpu().numpy()[~fits] == 0).all()


@pytest.mark.gpu
def test_window_flags_kernel(device):
    import torch

    s = systems.perovskite(3)
    builder = _gpu_builder(s.cell, 135, 6.0, 2.0, 1100, device)
    _, status = builder.build(torch.tensor(s.positions, device=device))
    wo = torch.zeros(1, dtype=torch.uint8, device=device)
    wc = torch.zeros(1, dtype=torch.uint8, device=device)
    we = torch.zeros(1, dtype=torch.int64, device=device)
    wi = torch.zeros(1, dtype=torch.int32, device=device)
    builder.accumulate_window(status, window_overflow=wo, window_capacity_overflow=wc, window_max_edges=we,
                              window_max_isolated=wi, check_isolated=True)
    assert (int(wo.item()), int(wc.item()), int(we.item()), int(wi.item())) == (0, 0, 2054, 0)
    small = _gpu_builder(s.cell, 135, 6.0, 2.0, 500, device)
    _, st2 = small.build(torch.tensor(s.positions, device=device))
    small.accumulate_window(st2, window_overflow=wo, window_capacity_overflow=wc, window_max_edges=we,
                            window_max_isolated=wi, check_isolated=True)
    assert (int(wo.item()), int(wc.item()), int(we.item())) == (1, 1, 2054)


@pytest.mark.gpu
@pytest.mark.parametrize("max_neighbors", [1, 8, 16, None])
def test_ragged_builder_growth_is_bitwise_identical(device, max_neighbors):
    """Forced tiny slot counts rebuild to the same graph (tests/test_ragged_builder_overflow.py:
    158-213 of the reference); the ragged rows equal the oracle's."""
    import torch

    from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder

    s = systems.perovskite(3)
    b = TensorGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers), atom_graph_cutoff=6.0,
                           line_graph_cutoff=None, max_neighbors=max_neighbors, device=device)
    g = b.build(torch.tensor(s.positions, device=device))
    assert max_neighbors is None or b.max_neighbors >= 20
    cell32 = s.cell.astype(F32)
    inv = b.inv_cell.cpu().numpy()
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    cand = onl.candidates(wrapped, cell32, F32((6.0 + 1e-6) ** 2), 640)
    ob = onl.build(s.positions, inv, cell32, cand, s.positions.astype(F32), wraps, F32(36.0), F32(1e-6),
                   (0, 0, 1), int(cand.num_neighbors.sum()))
    e = ob.n_edges
    ei = g.edge_index.cpu().numpy()
    assert int(g.n_edges.item()) == e == ei.shape[0]
    assert np.array_equal(ei[:, 0], ob.center[:e]) and np.array_equal(ei[:, 1], ob.neighbor[:e])
    assert np.array_equal(g.edge_image.cpu().numpy(), ob.images[:e].astype(F32))


# ------------------------------------------------------------------ line graph (three-body)
def _oracle_line(cell, positions, cutoff, skin, u_cap, t_cap, line_cutoff, inv=None):
    cell32 = cell.astype(F32)
    inv = _inv32(cell) if inv is None else inv
    _, wraps, wrapped = onl.wrap(positions, inv, cell32)
    bmax = onl.estimate_max_neighbors(cutoff + skin, safety_factor=2.0)
    cand = onl.candidates(wrapped, cell32, F32((cutoff + skin) ** 2), bmax)
    pad, _ = onl.self_loop_image(cell, cutoff)
    b = onl.build(positions, inv, cell32, cand, np.asarray(positions, dtype=F32), wraps, F32(cutoff * cutoff),
                  F32(skin + 1e-6), pad, 2 * u_cap, line2=F32(line_cutoff * line_cutoff))
    rev = onl.reverse(b.center, b.neighbor, b.images, b.edge_offsets, 2 * u_cap)
    lg = onl.line_graph(b, rev, positions.shape[0], 2 * u_cap, u_cap, t_cap, bmax)
    return cand, b, rev, lg, wrapped


def _edge_key(b, e):
    return (int(b.neighbor[e]), *map(int, b.images[e]))


@pytest.mark.parametrize("line_cutoff", [3.0, 3.5])
def test_oracle_line_graph_pinned(line_cutoff):
    """The oracle's pairs and triplets against independent formulations: the short-bond flags
    against FP64 distances (away from the cutoff), the triplet rows against the brute-force set
    of ordered bond pairs per centre, and the pair ids against their invariants (a row and its
    reverse share a pair, u2d is the lower row, leaders numbered in row order), plus the padding
    rule and the reference's capacity-boundary answers (tests/test_fixed_capacity_boundary.py:
    155-237): edges > or == e_capacity overflow, one padding pair leaves no overflow and takes
    every padding triplet."""
    s = systems.perovskite(3)
    cutoff, skin = 6.0, 2.0
    _, b0, _, _, wrapped = _oracle_line(s.cell, s.positions, cutoff, skin, 4096, 65536, line_cutoff)
    edges = b0.n_edges
    real_u = edges // 2
    d64 = np.linalg.norm(wrapped.astype(np.float64)[b0.neighbor[:edges]] + b0.images[:edges].astype(np.float64)
                         @ s.cell.astype(F32).astype(np.float64) - wrapped.astype(np.float64)[b0.center[:edges]], axis=1)
    far = np.abs(d64 - line_cutoff) > 1e-4
    assert np.array_equal(b0.short[:edges][far], (d64 < line_cutoff)[far])
    triplets = int(sum(int(c) * (int(c) - 1) for c in np.bincount(b0.center[:edges][b0.short[:edges]], minlength=135)))
    assert triplets > 0
    t_cap = triplets + 32
    for u_cap, expect in ((real_u - 1, True), (real_u, True), (real_u + 1, False)):
        _, b, rev, lg, _ = _oracle_line(s.cell, s.positions, cutoff, skin, u_cap, t_cap, line_cutoff)
        assert lg["overflow"] == expect
        line = lg["line_graph"].astype(np.int64)
        assert line[:, [1, 3]].max() < u_cap and line[:, [2, 4]].max() < 2 * u_cap and line.min() >= 0
        assert lg["d2u"].max() < u_cap and lg["u2d"].max() < 2 * u_cap
        if expect:
            lu = np.minimum(np.arange(t_cap) * u_cap // t_cap, u_cap - 1)
            assert np.array_equal(line[:, 1], lu) and np.array_equal(line[:, 2], 2 * lu)
            continue
        assert int(lg["pair_offsets"][-1]) == triplets and not lg["invalid_pairs"]
        # every padding triplet uses the single padding pair
        assert (line[triplets:, [1, 3]] == real_u).all() and (line[triplets:, [2, 4]] == edges).all()
        got = {(int(r[0]), _edge_key(b, r[2]), _edge_key(b, r[4])) for r in line[:triplets]}
        assert len(got) == triplets
        assert got == onl.triplet_set(b.center, b.neighbor, b.images, b.short, edges)
        assert all(b.center[r[2]] == r[0] and b.center[r[4]] == r[0] for r in line[:triplets])
        d2u, u2d = lg["d2u"].astype(np.int64), lg["u2d"].astype(np.int64)
        rows = np.arange(edges)
        assert np.array_equal(d2u[rows], d2u[rev[rows]])
        assert np.array_equal(u2d[d2u[rows]], np.minimum(rows, rev[rows]))
        leaders = rows[rows <= rev[rows]]
        assert np.array_equal(d2u[leaders], np.arange(real_u))
        pad_rows = np.arange(edges, 2 * u_cap)
        assert np.array_equal(d2u[pad_rows], np.minimum(real_u + (pad_rows - edges) // 2, u_cap - 1))
        assert np.array_equal(line[:triplets, 1], d2u[line[:triplets, 2]])
        # the angle -> bond CSR: row e's run holds exactly the triplets whose first bond is e
        eto = lg["edge_triplet_offsets"]
        assert eto[0] == 0 and (np.diff(eto) >= 0).all() and eto[-1] == triplets
        first = np.repeat(np.arange(len(eto) - 1), np.diff(eto))
        assert np.array_equal(first, line[:triplets, 2])
        # the second-bond CSR: row e's run through second_perm holds the triplets with e second
        sp = lg["second_perm"].astype(np.int64)
        assert np.array_equal(np.sort(sp[:triplets]), np.arange(triplets)) and (sp[triplets:] == -1).all()
        assert np.array_equal(line[sp[:triplets], 4], first)
        # the bond -> atom CSR: short_offsets over bond_rows lists each atom's short rows
        br, so = lg["bond_rows"].astype(np.int64), lg["short_offsets"]
        assert np.array_equal(br[:so[-1]], np.nonzero(b.short[:edges])[0]) and (br[so[-1]:] == -1).all()
        assert np.array_equal(b.center[br[:so[-1]]], np.repeat(np.arange(135), np.diff(so)))
    # triplets above t_capacity overflow too
    _, _, _, lg, _ = _oracle_line(s.cell, s.positions, cutoff, skin, real_u + 64, triplets - 1, line_cutoff)
    assert lg["overflow"]


def _gpu_line_builder(cell, n, cutoff, skin, u_cap, t_cap, line_cutoff, device):
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    return FixedCapacityGraphBuilder(cell=torch.tensor(cell, dtype=torch.float32), atomic_numbers=torch.ones(n),
                                     u_capacity=u_cap, t_capacity=t_cap, atom_graph_cutoff=cutoff,
                                     line_graph_cutoff=line_cutoff, candidate_cutoff=cutoff + skin,
                                     padding=PaddingRule("far_self_loops"), device=device)


def _assert_line_equal(builder, b, lg):
    assert np.array_equal(builder.short_flags.cpu().numpy().astype(bool), b.short)
    for name, buf in (("d2u", builder.directed2undirected), ("u2d", builder.undirected2directed),
                      ("short_counts", builder.short_counts), ("short_offsets", builder.short_offsets),
                      ("short_edge_matrix", builder.short_edge_matrix), ("pair_offsets", builder.pair_offsets),
                      ("line_graph", builder.line_graph), ("edge_triplet_offsets", builder.edge_triplet_offsets),
                      ("bond_rows", builder.bond_rows), ("second_perm", builder.second_perm)):
        assert np.array_equal(buf.cpu().numpy(), lg[name]), name
    assert bool(builder._invalid_pairs.item()) == lg["invalid_pairs"]
    assert bool(builder._overflow.item()) == lg["overflow"]
    assert builder.batch.triplets is builder.line_graph and builder.batch.pair_d2u is builder.directed2undirected


@pytest.mark.gpu
@pytest.mark.parametrize("n_atoms,line_cutoff", [(135, 3.5), (1080, 3.0), (5000, 3.0), (5000, 3.5), (10000, 3.5)])
def test_line_graph_builder_bit_exact(device, n_atoms, line_cutoff):
    """The HIP line graph (short-bond flags, undirected pairs, short lists, pair offsets, triplet
    rows, flags) bit-exact vs the oracle on the fused (<= 1 024 atoms) and multi-block builds
    (10 000 atoms: the pair scan's workgroup takes two passes of 8 192 atoms)."""
    import torch

    print(f"[line graph] n_atoms={n_atoms} cutoff={line_cutoff}", flush=True)
    s = systems.perovskite_atoms(n_atoms)
    cutoff, skin = 6.0, 2.0
    u_cap = int(round(15.3 * n_atoms / 2)) + 64
    t_cap = 40 * n_atoms
    builder = _gpu_line_builder(s.cell, n_atoms, cutoff, skin, u_cap, t_cap, line_cutoff, device)
    builder.build(torch.tensor(s.positions, dtype=torch.float64, device=device))
    inv = builder.inv_cell.cpu().numpy()
    cand, b, rev, lg, _ = _oracle_line(s.cell, s.positions, cutoff, skin, u_cap, t_cap, line_cutoff, inv=inv)
    torch.cuda.synchronize()
    assert np.array_equal(builder.center.cpu().numpy(), b.center)
    assert np.array_equal(builder.edge_reverse.cpu().numpy(), rev)
    _assert_line_equal(builder, b, lg)
    assert not lg["overflow"] and int(lg["pair_offsets"][-1]) > 0


@pytest.mark.gpu
def test_line_graph_builder_capacity_boundary(device):
    """The reference's boundary cases on the GPU (tests/test_fixed_capacity_boundary.py:155-237):
    edges > e_capacity and == e_capacity overflow (all-loop topology), one padding pair does not,
    triplets > t_capacity overflow; every index in range; bit-exact vs the oracle throughout."""
    import torch

    s = systems.perovskite(3)
    cutoff, skin, lc = 6.0, 2.0, 3.5
    _, b0, _, _, _ = _oracle_line(s.cell, s.positions, cutoff, skin, 4096, 65536, lc)
    real_u = b0.n_edges // 2
    triplets = int(sum(int(c) * (int(c) - 1) for c in np.bincount(b0.center[:b0.n_edges][b0.short[:b0.n_edges]],
                                                                  minlength=135)))
    for u_cap, t_cap, expect in ((real_u - 1, triplets + 32, True), (real_u, triplets + 32, True),
                                 (real_u + 1, triplets + 32, False), (real_u + 8, triplets - 1, True)):
        print(f"[line graph boundary] u_cap={u_cap} t_cap={t_cap}", flush=True)
        builder = _gpu_line_builder(s.cell, 135, cutoff, skin, u_cap, t_cap, lc, device)
        builder.build(torch.tensor(s.positions, device=device))
        inv = builder.inv_cell.cpu().numpy()
        _, b, rev, lg, _ = _oracle_line(s.cell, s.positions, cutoff, skin, u_cap, t_cap, lc, inv=inv)
        torch.cuda.synchronize()
        _assert_line_equal(builder, b, lg)
        assert lg["overflow"] == expect
        line = builder.line_graph.long()
        assert int(line[:, [1, 3]].max()) < u_cap and int(line[:, [2, 4]].max()) < 2 * u_cap
        assert int(line.min()) >= 0 and int(line[:, 0].max()) < 135
