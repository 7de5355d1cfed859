"""The fixed-capacity builder's three padding rules (fastmd/adapters/protocol.py:68-119):
far self-loops, exact-cutoff loops with the edge-vector override, and sink atoms
(fixed_capacity_builder.py:291-366, with a line graph :680-753 and the overflow topology
:1474-1513, 2163-2177). The oracle's rows are pinned on the CPU by the rules' invariants and
hand-reduced cases; the HIP builder equals the oracle bit for bit on the reference's capacity
boundaries (tests/test_fixed_capacity_boundary.py:155-237, 357-434), and a torch pair potential
with an exact cutoff gets exactly nothing from the padded rows under every rule."""
import numpy as np
import pytest

from oracle import nl as onl
from fastmd_amd import systems

F32 = np.float32
CUTOFF, SKIN = 5.0, 1.0


def _oracle_build(s, u_cap, n_dummy=0, pad_image=None, line_cutoff=None):
    cell32 = s.cell.astype(F32)
    inv = np.linalg.inv(cell32.astype(np.float64)).astype(F32)
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    bmax = onl.estimate_max_neighbors(CUTOFF + SKIN, safety_factor=2.0)
    cand = onl.candidates(wrapped, cell32, F32((CUTOFF + SKIN) ** 2), bmax)
    if pad_image is None:
        pad_image, _ = onl.self_loop_image(s.cell, CUTOFF)
    line2 = None if line_cutoff is None else F32(line_cutoff * line_cutoff)
    b = onl.build(s.positions, inv, cell32, cand, s.positions.astype(F32), wraps, F32(CUTOFF * CUTOFF),
                  F32(SKIN + 1e-6), pad_image, 2 * u_cap, line2=line2, n_dummy=n_dummy)
    return b, bmax


# ------------------------------------------------------------------------------------ CPU pins
def test_oracle_sink_rows_hand_reduced_and_invariants():
    """Sink padding of the oracle: every padded row a self-loop of a sink with image (3, 3, 3)
    and distance 1e6, the two rows of a padded pair on one sink, sinks in ascending order with
    as many pairs on each sink as the even split allows (one each when there are fewer pairs than
    sinks); real rows those of a far-loop build.
    Hand-reduced case: 5 free pairs over 2 sinks give the sinks n + (0, 0, 0, 1, 1)."""
    s = systems.perovskite(2)
    n = s.n_atoms
    loops, _ = _oracle_build(s, 4096)
    edges = loops.n_edges
    real_u = edges // 2
    for free_u, n_dummy in ((5, 2), (37, 4), (3, 8)):
        b, _ = _oracle_build(s, real_u + free_u, n_dummy=n_dummy)
        e_cap = 2 * (real_u + free_u)
        assert b.n_edges == edges and not b.overflow
        assert np.array_equal(b.center[:edges], loops.center[:edges])
        assert np.array_equal(b.images[:edges], loops.images[:edges])
        c, nb = b.center[edges:].astype(np.int64), b.neighbor[edges:].astype(np.int64)
        assert np.array_equal(c, nb) and (c >= n).all() and (c < n + n_dummy).all()
        assert (b.images[edges:] == 3).all() and (b.distances[edges:] == F32(1e6)).all()
        pairs = c.reshape(-1, 2) if (e_cap - edges) % 2 == 0 else None
        if pairs is not None:
            assert (pairs[:, 0] == pairs[:, 1]).all()
        assert (np.diff(c) >= 0).all()
        per_sink = np.bincount(c[::2] - n, minlength=n_dummy)
        if free_u >= n_dummy:  # every sink holds floor or ceil(free_u / n_dummy) pairs
            assert per_sink.min() >= free_u // n_dummy and per_sink.max() <= -(-free_u // n_dummy)
        else:  # fewer pairs than sinks: one pair per sink
            assert per_sink.max() == 1
        if (free_u, n_dummy) == (5, 2):
            assert np.array_equal(c[::2] - n, [0, 0, 0, 1, 1])


def test_oracle_override_and_exact_loop_rows():
    """Exact-cutoff padding: image-0 self-loops round robin over the real atoms (the far-loop rows
    with image 0) and the override holding the pad vector on the padded rows only."""
    s = systems.perovskite(2)
    n = s.n_atoms
    loops, _ = _oracle_build(s, 4096)
    edges = loops.n_edges
    b, _ = _oracle_build(s, edges // 2 + 40, pad_image=(0, 0, 0))
    e_cap = 2 * (edges // 2 + 40)
    assert np.array_equal(b.center[edges:], np.arange(e_cap - edges) % n)
    assert (b.images[edges:] == 0).all()
    ov = onl.pad_override(edges, e_cap, (CUTOFF, 0.0, 0.0))
    assert (ov[:edges] == 0).all() and (ov[edges:] == F32([CUTOFF, 0.0, 0.0])).all()
    assert (onl.pad_override(e_cap + 5, e_cap, (1.0, 2.0, 3.0)) == 0).all()  # overflow: no padded row


def test_self_loop_padding_refuses_an_inner_pad_vector():
    """The exact-cutoff pad vector must not lie inside the cutoff (fixed_capacity_builder.py:1008-1014)."""
    import torch

    from fastmd_amd.adapters.protocol import PaddingRule
    from fastmd_amd.graph.fixed_capacity_builder import self_loop_padding

    cell = torch.eye(3) * 12.0
    assert self_loop_padding(PaddingRule("exact_rc_loops"), cell, CUTOFF) == ((0, 0, 0), CUTOFF,
                                                                              (CUTOFF, 0.0, 0.0))
    for vector in ((1.0, 0.0, 0.0), (0.0, 0.0, 0.0)):
        with pytest.raises(ValueError, match="shorter than the cutoff"):
            self_loop_padding(PaddingRule("exact_rc_loops", pad_vector=vector), cell, CUTOFF)
    with pytest.raises(ValueError, match="no self-loops"):
        self_loop_padding(PaddingRule("sink_atoms"), cell, CUTOFF)


@pytest.mark.parametrize("n_dummy", [0, 3])
def test_oracle_line_graph_padding_and_overflow_topology(n_dummy):
    """With a line graph: padding triplets on the single padding pair (one free pair) and, for
    sinks, on sink atoms spread in ascending order; an overflowed build's published rows and
    triplets are the all-loop (u mod n) or all-sink topology with image +/- the pad image
    (+/- 3 for sinks) by row parity; every index in range."""
    s = systems.perovskite(2)
    n = s.n_atoms
    lc = 3.5
    b0, bmax = _oracle_build(s, 4096, line_cutoff=lc)
    edges = b0.n_edges
    real_u = edges // 2
    short = b0.short[:edges]
    triplets = int(sum(int(c) * (int(c) - 1) for c in np.bincount(b0.center[:edges][short], minlength=n)))
    pad_image, _ = onl.self_loop_image(s.cell, CUTOFF)
    for u_cap, t_cap, expect in ((real_u + 1, triplets + 32, False), (real_u, triplets + 32, True),
                                 (real_u + 8, triplets - 1, True)):
        b, _ = _oracle_build(s, u_cap, n_dummy=n_dummy, line_cutoff=lc)
        rev = onl.reverse(b.center, b.neighbor, b.images, b.edge_offsets, 2 * u_cap)
        lg = onl.line_graph(b, rev, n, 2 * u_cap, u_cap, t_cap, bmax, n_dummy=n_dummy, pad_image=pad_image)
        assert lg["overflow"] == expect
        line = lg["line_graph"].astype(np.int64)
        n_all = n + n_dummy
        assert line.min() >= 0 and line[:, 0].max() < n_all
        assert line[:, [1, 3]].max() < u_cap and line[:, [2, 4]].max() < 2 * u_cap
        assert lg["center"].max() < n_all and lg["center"].min() >= 0
        if not expect:
            assert (line[triplets:, [1, 3]] == real_u).all() and (line[triplets:, [2, 4]] == edges).all()
            atoms = line[triplets:, 0]
            if n_dummy:
                assert (atoms >= n).all() and (np.diff(atoms) >= 0).all()
                assert set(atoms.tolist()) == set(range(n, n + n_dummy))
            else:
                assert (atoms == 0).all()  # the atom of the first (here the only) padding pair
            assert np.array_equal(lg["center"], b.center)
            continue
        e = np.arange(2 * u_cap)
        if n_dummy:
            assert (line[:, 0] >= n).all() and (lg["center"] >= n).all()
            expect_atom = n + (e // 2) * n_dummy // u_cap
            expect_image = np.where(e % 2 == 0, 3, -3)[:, None] * np.ones(3, np.int64)
        else:
            expect_atom = (e // 2) % n
            expect_image = np.where(e % 2 == 0, 1, -1)[:, None] * np.asarray(pad_image)
        assert np.array_equal(lg["center"], expect_atom) and np.array_equal(lg["neighbor"], expect_atom)
        assert np.array_equal(lg["images"], expect_image)
        assert np.array_equal(line[:, 0], lg["center"][line[:, 2]])  # a triplet sits on its pair's atom


# ------------------------------------------------------------------------------------ GPU parity
RULES = ("far_self_loops", "exact_rc_loops", "sink_atoms")


def _rule(kind):
    from fastmd_amd.adapters.protocol import PaddingRule

    return PaddingRule(kind)


def _gpu_builder(s, u_cap, kind, device, n_dummy=16, t_cap=0, line_cutoff=None):
    import torch

    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    return FixedCapacityGraphBuilder(cell=torch.tensor(s.cell, dtype=torch.float32),
                                     atomic_numbers=torch.tensor(s.numbers), u_capacity=u_cap, t_capacity=t_cap,
                                     atom_graph_cutoff=CUTOFF, line_graph_cutoff=line_cutoff,
                                     candidate_cutoff=CUTOFF + SKIN, padding=_rule(kind), n_dummy=n_dummy,
                                     device=device)


@pytest.mark.gpu
@pytest.mark.parametrize("n_cells", [3, (6, 6, 6)])
@pytest.mark.parametrize("kind", RULES)
def test_edges_only_padding_rules_bit_exact(device, kind, n_cells):
    """Edges-only builds at the capacity boundary (edges above, equal to and 40 pairs below
    e_capacity; the last pads more rows than there are atoms, so the round robin wraps) on the
    fused (135 atoms) and multi-block (1 080) paths: rows, published buffers, distances, sink
    rows and override bit-exact vs the oracle; every index within the real and sink rows."""
    import torch

    print(f"[padding] {kind} cells={n_cells}", flush=True)
    s = systems.perovskite(n_cells, sigma=0.1)
    n = s.n_atoms
    loops, _ = _oracle_build(s, 10 ** 6)
    edges = loops.n_edges
    n_dummy = 16 if kind == "sink_atoms" else 0
    for u_cap, expect in ((edges // 2 - 1, True), (edges // 2, False), (edges // 2 + 40 + n, False)):
        builder = _gpu_builder(s, u_cap, kind, device)
        _, status = builder.build(torch.tensor(s.positions, device=device))
        pad = (0, 0, 0) if kind == "exact_rc_loops" else None
        b, _ = _oracle_build(s, u_cap, n_dummy=n_dummy, pad_image=pad)
        torch.cuda.synchronize()
        assert int(status.edge_count.item()) == edges and bool(status.overflow.item()) == expect == b.overflow
        assert np.array_equal(builder.center.cpu().numpy(), b.center)
        assert np.array_equal(builder.neighbor.cpu().numpy(), b.neighbor)
        assert np.array_equal(builder.images.cpu().numpy(), b.images)
        ec = min(edges, 2 * u_cap)
        dist = builder.distances.cpu().numpy()
        assert np.array_equal(dist[:ec], b.distances[:ec])
        if kind == "sink_atoms":
            assert (dist[ec:] == F32(1e6)).all()
        batch = builder.batch
        ei = batch.edge_index.cpu().numpy()
        assert np.array_equal(ei[:, 0], b.center) and np.array_equal(ei[:, 1], b.neighbor)
        assert np.array_equal(batch.edge_image.cpu().numpy(), b.images.astype(F32))
        assert ei.min() >= 0 and ei.max() < n + n_dummy
        assert batch.positions.shape == (n + n_dummy, 3) and batch.species.shape == (n + n_dummy,)
        if n_dummy:
            assert not bool(batch.positions[n:].any()) and bool((batch.species[n:] == 1).all())
        if kind == "exact_rc_loops":
            ov = onl.pad_override(edges, 2 * u_cap, (CUTOFF, 0.0, 0.0))
            assert np.array_equal(batch.edge_vec_override.cpu().numpy(), ov)
        else:
            assert batch.edge_vec_override is None


@pytest.mark.gpu
@pytest.mark.parametrize("n_dummy", [0, 3])
def test_line_graph_padding_and_overflow_topology_bit_exact(device, n_dummy):
    """A line-graph builder with far self-loop or sink padding on the reference's boundary cases
    (one free pair, no free pair, triplets above t_capacity): pairs, triplets, flags and the
    published rows (the all-padding topology on overflow) bit-exact vs the oracle."""
    import torch

    print(f"[padding] line graph n_dummy={n_dummy}", flush=True)
    s = systems.perovskite(3, sigma=0.1)
    n = s.n_atoms
    lc = 3.5
    b0, bmax = _oracle_build(s, 10 ** 6, line_cutoff=lc)
    edges = b0.n_edges
    real_u = edges // 2
    triplets = int(sum(int(c) * (int(c) - 1)
                       for c in np.bincount(b0.center[:edges][b0.short[:edges]], minlength=n)))
    pad_image, _ = onl.self_loop_image(s.cell, CUTOFF)
    kind = "sink_atoms" if n_dummy else "far_self_loops"
    for u_cap, t_cap in ((real_u + 1, triplets + 32), (real_u, triplets + 32), (real_u + 8, triplets - 1),
                         (real_u - 1, triplets + 32)):
        builder = _gpu_builder(s, u_cap, kind, device, n_dummy=max(n_dummy, 1), t_cap=t_cap, line_cutoff=lc)
        builder.build(torch.tensor(s.positions, device=device))
        b, _ = _oracle_build(s, u_cap, n_dummy=n_dummy, line_cutoff=lc)
        rev = onl.reverse(b.center, b.neighbor, b.images, b.edge_offsets, 2 * u_cap)
        lg = onl.line_graph(b, rev, n, 2 * u_cap, u_cap, t_cap, bmax, n_dummy=n_dummy, pad_image=pad_image)
        torch.cuda.synchronize()
        assert bool(builder._overflow.item()) == lg["overflow"]
        for name, buf in (("d2u", builder.directed2undirected), ("u2d", builder.undirected2directed),
                          ("pair_offsets", builder.pair_offsets), ("line_graph", builder.line_graph),
                          ("center", builder.center), ("neighbor", builder.neighbor), ("images", builder.images)):
            assert np.array_equal(buf.cpu().numpy(), lg[name]), (u_cap, t_cap, name)
        ei = builder.batch.edge_index.cpu().numpy()
        assert np.array_equal(ei[:, 0], lg["center"])
        assert np.array_equal(builder.batch.edge_image.cpu().numpy(), lg["images"].astype(F32))


@pytest.mark.gpu
@pytest.mark.parametrize("kind", RULES)
def test_padding_rules_add_nothing(device, kind):
    """A torch pair potential with an exact cutoff through the engine derivative: energy and
    forces of a padded batch equal those of its real rows alone, and the padded rows alone give
    exactly zero energy and forces; the three rules give the same energy."""
    import dataclasses

    import torch
    from torch_pair_adapter import TorchPairAdapter

    from fastmd_amd.engine.energy_derivative import EnergyDerivative

    s = systems.perovskite(3, sigma=0.15)
    n = s.n_atoms
    adapter = TorchPairAdapter(_rule(kind), device=device)
    loops, _ = _oracle_build(s, 10 ** 6)
    edges = loops.n_edges
    builder = _gpu_builder(s, edges // 2 + 37, kind, device)
    builder.build(torch.tensor(s.positions, device=device))
    batch = builder.batch
    deriv = EnergyDerivative(adapter)
    full = deriv(batch, adapter.prepare(batch), n_real=n)
    ov = batch.edge_vec_override
    real = dataclasses.replace(batch, edge_index=batch.edge_index[:edges], edge_image=batch.edge_image[:edges],
                               edge_vec_override=None if ov is None else ov[:edges])
    alone = deriv(real, real, n_real=n)
    pad = dataclasses.replace(batch, edge_index=batch.edge_index[edges:], edge_image=batch.edge_image[edges:],
                              n_edges=torch.zeros_like(batch.n_edges),
                              edge_vec_override=None if ov is None else ov[edges:])
    nothing = deriv(pad, pad, n_real=n)
    torch.cuda.synchronize()
    e_full, e_alone = float(full["e"].item()), float(alone["e"].item())
    assert abs(e_full - e_alone) <= 1e-12 * abs(e_alone) and abs(e_alone) > 0.05
    assert torch.allclose(full["f"][0][:n], alone["f"][0][:n], rtol=0, atol=1e-6)
    assert float(nothing["e"].item()) == 0.0 and float(nothing["f"][0].abs().max()) == 0.0
    ref = EnergyDerivative(TorchPairAdapter(device=device))
    far = _gpu_builder(s, edges // 2 + 37, "far_self_loops", device)
    far.build(torch.tensor(s.positions, device=device))
    e_far = float(ref(far.batch, far.batch, n_real=n)["e"].item())
    assert abs(e_full - e_far) <= 1e-12 * abs(e_far)


@pytest.mark.gpu
def test_sink_padded_model_runs_whole_step_md(device):
    """GPU-resident MD of the torch pair potential with sink padding (whole-step graphs, the
    sink rows in every build) follows the far-self-loop run: positions within 1e-5 A and
    energies within 1e-9 relative after 40 steps; the HIP models refuse a sink-padded batch."""
    import torch
    from torch_pair_adapter import TorchPairAdapter

    from fastmd_amd.config import InferenceConfig
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics
    from fastmd_amd.models.pair_potential import MorsePairAdapter

    s = systems.perovskite(3)
    p0 = maxwell_boltzmann_momenta(s.masses, 600.0, 3)
    runs = {}
    for kind in ("sink_atoms", "far_self_loops"):
        md = GPUResidentMolecularDynamics(s, model=TorchPairAdapter(_rule(kind), device=device), device=device,
                                          temperature=600.0, timestep=0.5, tdamp=25.0, momenta=p0,
                                          steps_per_launch=5, config=InferenceConfig(execution="whole_step"))
        md.run(40)
        torch.cuda.synchronize()
        runs[kind] = (md.integrator.positions.clone(), float(md.integrator.potential_energy.item()))
        if kind == "sink_atoms":
            assert md.whole_step_runner is not None
            assert md.whole_step_runner.builder.batch.positions.shape[0] == s.n_atoms + 64
    (q_sink, e_sink), (q_far, e_far) = runs["sink_atoms"], runs["far_self_loops"]
    assert float((q_sink - q_far).abs().max()) < 1e-5
    assert abs(e_sink - e_far) <= 1e-9 * abs(e_far)
    sink = _gpu_builder(s, 1200, "sink_atoms", device)
    sink.build(torch.tensor(s.positions, device=device))
    with pytest.raises(ValueError, match="sink rows"):
        MorsePairAdapter(device=device).prepare(sink.batch)
