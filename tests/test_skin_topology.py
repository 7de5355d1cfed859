"""Skin-topology reuse (fastmd/execution/skin_topology.py:97-442): fixed-frame energies and forces of
one system whose candidate list is kept across calls, against the CPU oracle and against fresh
per-call builds."""
import dataclasses

import numpy as np
import pytest

from fastmd_amd import systems


def _adapter(name, device):
    if name == "morse":
        from fastmd_amd.models.pair_potential import MorsePairAdapter

        return MorsePairAdapter(device=device)
    from fastmd_amd.models.mace_like import MaceLikeAdapter

    return MaceLikeAdapter(device=device)


def _oracle(name, s):
    import md_oracle

    if name == "morse":
        return md_oracle.morse_forces(s)
    from fastmd_amd.models.mace_like import MaceLike, MaceLikeConfig

    params = {k: v.detach().clone() for k, v in MaceLike(MaceLikeConfig()).named_parameters()}
    return md_oracle.mace_like_forces(s, params, dataclasses.asdict(MaceLikeConfig()))


def _walk(s, calls, seed, step=0.12, keep=0.8):
    """Coordinates of successive calls: each atom's offset from its lattice site follows
    u <- keep u + N(0, step) (stationary rms step / sqrt(1 - keep^2), 0.2 A: a thermal-like
    configuration), and every third call is handed in wrapped by random lattice vectors (ASE's
    atoms.wrap() between calls)."""
    rng = np.random.default_rng(seed)
    u = np.zeros_like(s.positions)
    out = []
    for k in range(calls):
        u = keep * u + rng.normal(0, step, u.shape)
        shown = s.positions + u
        if k % 3 == 2:
            shown = shown + rng.integers(-1, 2, size=u.shape) @ s.cell
        out.append(shown)
    return out


def _fresh(adapter, s, positions, u_cap, device, t_cap=0):
    """A fresh refresh + build of capacity (u_cap, t_cap) and the engine derivative, eagerly."""
    import torch

    from fastmd_amd.engine.energy_derivative import engine_derivative
    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    line = dict(line_graph_cutoff=None, t_capacity=0) if not t_cap else dict(line_graph_cutoff=adapter.topology_spec().triplet_cutoff, t_capacity=t_cap)
    b = FixedCapacityGraphBuilder(cell=torch.tensor(s.cell, dtype=torch.float32),
                                  atomic_numbers=torch.tensor(s.numbers), u_capacity=u_cap, atom_graph_cutoff=6.0,
                                  candidate_cutoff=8.0, minimum_image=True, device=device,
                                  padding=adapter.padding_rule(), prepare=adapter.prepare, **line)
    graph, _ = b.build(torch.tensor(positions, dtype=torch.float32, device=device), rebuild_candidates=True)
    out = engine_derivative(adapter)(b.batch, graph, task="ef", n_real=s.n_atoms)
    return float(out["e"].reshape(-1)[0]), out["f"][0][: s.n_atoms].cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["morse", "mace_like"])
def test_skin_topology_matches_oracle_and_fresh_builds(device, name):
    """Over 30 calls of a thermal-like walk (lattice-wrapped coordinates every third call): energies
    within 1e-5 eV/atom and forces within 1e-4 eV/A of the oracle; each call bitwise equal to a
    fresh candidate refresh + build of the same capacity; the captured and the eager runner
    bitwise equal; candidates refreshed only when an atom moved 0.45 of the skin."""
    from fastmd_amd.execution.skin_topology import SkinTopologyRunner

    print(f"[skin topology] {name}", flush=True)
    s = systems.perovskite(3)
    adapter = _adapter(name, device)
    oracle = _oracle(name, s)
    graphs = SkinTopologyRunner(adapter, atomic_numbers=s.numbers, cell=s.cell, device=device)
    eager = SkinTopologyRunner(adapter, atomic_numbers=s.numbers, cell=s.cell, device=device, capture=False)
    for k, q in enumerate(_walk(s, 30, seed=4)):
        got = graphs.evaluate(q)
        same = eager.evaluate(q)
        assert got["e"] == same["e"] and np.array_equal(got["f"], same["f"]), k
        f_ref, e_ref = oracle(q)
        assert abs(got["e"] - e_ref) < 1e-5 * s.n_atoms, (k, got["e"], e_ref)
        assert np.abs(got["f"] - f_ref).max() < 1e-4, k
        e_fresh, f_fresh = _fresh(adapter, s, q, graphs.last_bucket[0], device)
        assert got["e"] == e_fresh and np.array_equal(got["f"], f_fresh), k
    st = graphs.stats()
    print(f"[skin topology] {name}: {st}", flush=True)
    assert st["calls"] == 30 and 2 <= st["refreshes"] <= 12 and st["redo_skin"] == 0
    assert st["refreshes"] == eager.stats()["refreshes"]


@pytest.mark.gpu
def test_skin_topology_three_body_line_graph(device):
    """A line-graph model (configs[4]'s three-body model, 3.5 A bonds): each call of a thermal-like
    walk bitwise equal to a fresh line-graph build of its bucket, captured == eager."""
    from fastmd_amd.execution.skin_topology import SkinTopologyRunner
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter, ThreeBodyConfig

    s = systems.perovskite(3)
    adapter = ThreeBodyAdapter(config=ThreeBodyConfig(bond_cutoff=3.5), device=device)
    graphs = SkinTopologyRunner(adapter, atomic_numbers=s.numbers, cell=s.cell, device=device, t_step=512)
    eager = SkinTopologyRunner(adapter, atomic_numbers=s.numbers, cell=s.cell, device=device, t_step=512,
                               capture=False)
    for k, q in enumerate(_walk(s, 12, seed=6)):
        got = graphs.evaluate(q)
        same = eager.evaluate(q)
        assert got["e"] == same["e"] and np.array_equal(got["f"], same["f"]), k
        e_fresh, f_fresh = _fresh(adapter, s, q, graphs.last_bucket[0], device, t_cap=graphs.last_bucket[1])
        assert got["e"] == e_fresh and np.array_equal(got["f"], f_fresh), k
    st = graphs.stats()
    print(f"[skin topology] three-body: {st}", flush=True)
    assert st["last_triplet_count"] > 0 and st["calls"] == 12


@pytest.mark.gpu
def test_skin_topology_device_check_and_capacity_redo(device, monkeypatch):
    """With the host's proactive refresh switched off, the device's skin test catches a stale list
    (the call is redone after a refresh, results still the oracle's); a bucket without room for
    the demand is redone in a larger one."""
    from fastmd_amd.execution import skin_topology as st

    s = systems.perovskite(3)
    adapter = _adapter("morse", device)
    oracle = _oracle("morse", s)
    monkeypatch.setattr(st, "PROACTIVE_REFRESH_FRACTION", 100.0)
    runner = st.SkinTopologyRunner(adapter, atomic_numbers=s.numbers, cell=s.cell, device=device, u_step=8,
                                   min_pad_u=1)
    runner._factors = (1.0, 1.0)  # no thermal headroom: a bucket leaves at most 9 pairs free
    runner.evaluate(s.positions)
    q = s.positions + np.random.default_rng(9).normal(0, 0.7, s.positions.shape)  # some atom > skin / 2
    got = runner.evaluate(q)
    # a disordered configuration (pairs at 2 A, force curvature ~60 eV/A^2): the float32 geometry
    # alone moves forces by 1e-4 eV/A against the float64 oracle, so the call is checked bitwise
    # against a fresh build of its bucket, and its energy against the oracle
    e_fresh, f_fresh = _fresh(adapter, s, q, runner.last_bucket[0], device)
    assert runner.redo_skin == 1 and runner.refreshes == 2
    assert got["e"] == e_fresh and np.array_equal(got["f"], f_fresh)
    assert abs(got["e"] - oracle(q)[1]) < 1e-5 * s.n_atoms
    # pull the atoms around the cell's centre up to 0.8 A closer to it (below the refresh
    # threshold): 13 more pairs, more than the bucket's slack of at most 9
    before = runner.last_edge_count
    v = s.cell.sum(0) / 2 - q
    d = np.linalg.norm(v, axis=1)
    q2 = q + (0.8 * np.clip(d / 8, 0, 1) * (d < 12))[:, None] * v / d[:, None]
    got = runner.evaluate(q2)
    e_fresh, f_fresh = _fresh(adapter, s, q2, runner.last_bucket[0], device)
    assert runner.last_edge_count > before
    assert runner.redo_capacity >= 1
    assert got["e"] == e_fresh and np.array_equal(got["f"], f_fresh)
    assert abs(got["e"] - oracle(q2)[1]) < 1e-5 * s.n_atoms
