"""(f) The whole MD step as a hipGraph: replays equal the eager MD bitwise (the reference's own
check with a deterministic pair potential, tests/test_fixed_capacity_boundary.py:497-536), also
through capacity growth (recapture) and candidate refresh / fallback windows; the MD is
checked against the CPU oracle (NHC + Morse) over many steps."""
import numpy as np
import pytest

from fastmd_amd import systems
from fastmd_amd.config import CapacityConfig, InferenceConfig


def test_inference_config_contract():
    assert InferenceConfig().resolved_execution == "whole_step"
    assert InferenceConfig(execution="eager").resolved_execution == "eager"
    assert InferenceConfig(execution="model_graph").resolved_execution == "model_graph"
    with pytest.raises(ValueError):
        InferenceConfig(execution="fast")
    with pytest.raises(ValueError):
        CapacityConfig(u_step=0)
    with pytest.raises(ValueError):
        CapacityConfig(candidate_skin=-1.0)


def test_capacity_tiers_known_answers():
    from fastmd_amd.engine.capacity_policy import JointCapacityPolicy, held_demand, tier, whole_step_headroom

    assert tier(1000, 512, 256) == 1536 and tier(1100, 512, 256) == 1536 and tier(1300, 512, 256) == 2048
    assert held_demand(1000, 8, 1.0) == 1008 and held_demand(1000, 8, 1.02) == 1020
    assert whole_step_headroom(77000, 32) == 576 and whole_step_headroom(1027, 32) == 0
    p = JointCapacityPolicy(u_step=32, min_pad_u=32)
    k = p.start(held_demand(1027, 0, 1.02))
    assert k.u_capacity == 1088  # 135-atom perovskite (1 027 undirected edges), MACE capacity step
    assert p.grow(k, 900).u_capacity == 1088 and p.grow(k, 1100).u_capacity > 1088
    # joint tiers: pairs and triplets each take their own tier, growth keeps the larger of each
    j = JointCapacityPolicy(u_step=128, min_pad_u=128, t_step=128, min_pad_t=128)
    k = j.start(1040, 980)
    assert (k.u_capacity, k.t_capacity) == (1280, 1152)
    g = j.grow(k, 1000, 1100)
    assert (g.u_capacity, g.t_capacity) == (1280, 1280) and j.capacity_history == [k, g]


def _md(model, execution, device, steps_per_launch=1, capacity=None, system=None, temperature=500.0):
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics

    s = system or systems.perovskite(3)
    return GPUResidentMolecularDynamics(s, model=model, device=device, temperature=temperature, timestep=0.25,
                                        tdamp=25.0, config=InferenceConfig(execution=execution,
                                                                           capacity=capacity or CapacityConfig()),
                                        steps_per_launch=steps_per_launch)


def _adapter(model_name, device, bond_cutoff=3.5):
    from fastmd_amd.models.mace_like import MaceLikeAdapter
    from fastmd_amd.models.pair_potential import MorsePairAdapter
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter, ThreeBodyConfig

    if model_name == "morse":
        return MorsePairAdapter(device=device)
    if model_name == "mace_like":
        return MaceLikeAdapter(device=device)
    return ThreeBodyAdapter(config=ThreeBodyConfig(bond_cutoff=bond_cutoff), device=device)


def _state(md):
    import torch

    torch.cuda.synchronize()
    return md.integrator.state.flat.detach().cpu().clone()


@pytest.mark.gpu
@pytest.mark.parametrize("model_name", ["morse", "mace_like", "threebody"])
@pytest.mark.parametrize("steps_per_launch", [1, 5])
def test_whole_step_equals_eager_bitwise(device, model_name, steps_per_launch):
    import torch

    print(f"[whole_step] {model_name} spl={steps_per_launch}", flush=True)
    make = lambda: _adapter(model_name, device)  # noqa: E731
    eager = _md(make(), "eager", device)
    graph = _md(make(), "whole_step", device, steps_per_launch=steps_per_launch)
    assert torch.equal(_state(eager), _state(graph))
    eager.run(20)
    graph.run(20)
    a, b = _state(eager), _state(graph)
    assert torch.equal(a, b), float((a - b).abs().max())
    stats = graph.whole_step_stats()
    assert stats["launches"] == 20 // steps_per_launch and stats["fallback_windows"] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("k", [15, 20])
def test_whole_step_equals_eager_bitwise_configs3_sizes(device, k):
    """configs[3]'s largest supercells (16 875 and 40 000 atoms), MACE-like model: 20 whole-step
    steps (windows of 10) give the eager trajectory bitwise, on the large-grid kernel paths."""
    import torch

    print(f"[whole_step configs3] k={k}", flush=True)
    s = systems.perovskite(k)
    eager = _md(_adapter("mace_like", device), "eager", device, system=s)
    graph = _md(_adapter("mace_like", device), "whole_step", device, steps_per_launch=10, system=s)
    eager.run(20)
    graph.run(20)
    a, b = _state(eager), _state(graph)
    assert torch.equal(a, b), float((a - b).abs().max())
    assert graph.whole_step_stats()["launches"] == 2


@pytest.mark.gpu
def test_whole_step_capacity_growth_and_refresh_paths(device):
    """A tiny capacity step forces overflow -> growth -> recapture; a tiny skin forces candidate
    refreshes and fallback windows. The trajectory stays the eager one, bitwise."""
    import torch

    from fastmd_amd.models.pair_potential import MorsePairAdapter

    s = systems.perovskite(3)
    eager = _md(MorsePairAdapter(device=device), "eager", device, system=s)
    tight = CapacityConfig(u_step=1, min_pad_u=0, candidate_skin=0.05)
    graph = _md(MorsePairAdapter(device=device), "whole_step", device, steps_per_launch=2, capacity=tight, system=s)
    eager.run(30)
    graph.run(30)
    assert torch.equal(_state(eager), _state(graph))
    st = graph.whole_step_stats()
    print(st, flush=True)
    assert st["candidate_refreshes"] > 2


@pytest.mark.gpu
@pytest.mark.parametrize("model_name", ["morse", "mace_like", "threebody"])
def test_model_graph_equals_eager_bitwise(device, model_name):
    """The model_graph mode (the model's forward + VJP replayed per capacity bucket, the ragged
    build and the integrator eager) gives the eager trajectory bitwise; a tiny capacity step makes
    the heating system leave its first bucket (new captures; smaller buckets reused)."""
    import torch

    print(f"[model_graph] {model_name}", flush=True)
    tight = CapacityConfig(u_step=8, min_pad_u=0, t_step=8, min_pad_t=0, warmup=1)
    s = systems.perovskite(3)
    eager = _md(_adapter(model_name, device), "eager", device, system=s, temperature=3000.0)
    graph = _md(_adapter(model_name, device), "model_graph", device, capacity=tight, system=s, temperature=3000.0)
    assert torch.equal(_state(eager), _state(graph))
    eager.run(60)
    graph.run(60)
    a, b = _state(eager), _state(graph)
    assert torch.equal(a, b), float((a - b).abs().max())
    st = graph.model_graph_stats()
    print(st, flush=True)
    assert st["replays"] == 61 and st["captures"] >= 2
    f_eager, e_eager = eager.evaluate()
    f_graph, e_graph = graph.evaluate()
    assert torch.equal(f_eager, f_graph) and torch.equal(e_eager, e_graph)


@pytest.mark.gpu
def test_whole_step_threebody_triplet_capacity_growth(device):
    """Triplet tiers of one triplet (a model whose capacity step is 1 / 0 / 1.0) with the bond
    cutoff at the B-X distance (3.1 A, where bonds come and go at 3000 K): windows overflow their
    triplets, the capacity grows and the step is recaptured; the trajectory stays the eager one,
    bitwise."""
    import torch

    from fastmd_amd.adapters.protocol import CapacityStep
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter, ThreeBodyConfig

    class Tight(ThreeBodyAdapter):
        def capacity_step(self):
            return CapacityStep(u_step=1, min_pad_u=0, u_thermal_factor=1.0, t_step=1, min_pad_t=0,
                                t_thermal_factor=1.0)

    s = systems.perovskite(3)
    cfg = ThreeBodyConfig(bond_cutoff=3.1)
    eager = _md(Tight(config=cfg, device=device), "eager", device, system=s, temperature=3000.0)
    graph = _md(Tight(config=cfg, device=device), "whole_step", device, steps_per_launch=2, system=s,
                temperature=3000.0)
    eager.run(200)
    graph.run(200)
    a, b = _state(eager), _state(graph)
    assert torch.equal(a, b), float((a - b).abs().max())
    st = graph.whole_step_stats()
    print(st, flush=True)
    assert len(st["triplet_capacity_history"]) > 1
    assert st["triplet_capacity_history"] == sorted(st["triplet_capacity_history"])


@pytest.mark.gpu
@pytest.mark.parametrize("model_name", ["morse", "mace_like", "threebody"])
def test_windows_launched_behind_match_settled_windows_bitwise(device, model_name, monkeypatch):
    """run() launches each next window before the host reads the flags of the one in flight. With
    a launch behind EVERY window (refresh_unlikely forced true) and a tiny skin and capacity step
    (candidate refreshes, fallbacks and a capacity growth behind which windows were launched),
    the rollbacks (drop to the window's end, rewind to its start) give the trajectory of windows
    settled one at a time, bitwise."""
    import torch

    from fastmd_amd.execution.whole_step_cuda_graph import WholeStepGraphRunner

    print(f"[launch behind] {model_name}", flush=True)
    make = lambda: _adapter(model_name, device)  # noqa: E731
    s = systems.perovskite(3)
    tight = CapacityConfig(u_step=1, min_pad_u=0, candidate_skin=0.05)
    settled = _md(make(), "whole_step", device, steps_per_launch=2, capacity=tight, system=s)
    settled.launch_behind = False
    settled.run(40)
    monkeypatch.setattr(WholeStepGraphRunner, "refresh_unlikely", lambda self: True)
    behind = _md(make(), "whole_step", device, steps_per_launch=2, capacity=tight, system=s)
    behind.run(40)
    a, b = _state(settled), _state(behind)
    assert torch.equal(a, b), float((a - b).abs().max())
    sa, sb = settled.whole_step_stats(), behind.whole_step_stats()
    print(sa, sb, flush=True)
    assert sb["windows_ahead"] >= 19 and sb["windows_rolled_back"] > 0 and sa["windows_ahead"] == 0
    for key in ("launches", "candidate_refreshes", "fallback_windows", "capacity_history"):
        assert sa[key] == sb[key], key


@pytest.mark.gpu
@pytest.mark.parametrize("execution", ["whole_step", "model_graph"])
def test_morse_md_matches_cpu_oracle(device, execution):
    """configs[0] plumbing: Morse MD (NHC 500 K, dt 0.25 fs) for 200 steps on the GPU, in the
    whole-step and in the model_graph mode, against the CPU oracle's integration (NumPy NHC,
    float64 Morse forces rounded to float32 like the GPU's, brute-force skin pair list): the
    trajectories coincide, so the positions agree to float32 noise and so does the conserved
    quantity at every sampled step (its change since step 0, which cancels the float32 rounding of
    the initial energy). The GPU's Morse energy is formed from float32 geometry (distances rounded
    at about 1e-6 A, pair forces up to 0.1 eV/A, 2 054 edges: about 1e-5 eV, 1e-7 eV/atom, measured
    1.4e-5 eV), the oracle's in float64, so the conserved quantities are held to 1e-6 eV/atom, a
    tenth of the north-star energy tolerance."""
    import md_oracle
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.models.pair_potential import MorsePairAdapter

    s = systems.perovskite(3)
    md = _md(MorsePairAdapter(device=device), execution, device, steps_per_launch=10, system=s)
    oracle = md_oracle.run_nhc(s, md_oracle.morse_forces(s), maxwell_boltzmann_momenta(s.masses, 500.0, 0), 200,
                               sample_every=10, positions_until=200)
    c0 = md.conserved_energy()
    assert abs(c0 - oracle["conserved"][0]) < 1e-6 * s.n_atoms
    dq, dc = [], []
    for k in range(1, 21):
        md.run(10)
        dq.append(float(np.abs(md.positions.cpu().numpy() - oracle["positions"][k]).max()))
        dc.append(abs((md.conserved_energy() - c0) - (oracle["conserved"][k] - oracle["conserved"][0])))
    print(f"[morse md {execution}] max |dq| {max(dq):.2e} A, max |dC| {max(dc):.2e} eV", flush=True)
    assert max(dq) < 1e-4, dq
    assert max(dc) < 1e-6 * s.n_atoms, dc


def test_oracle_morse_forces_match_the_torch_oracle():
    """The vectorized Morse forces of the MD oracle (tests/md_oracle.py) against the oracle's
    autograd Morse (oracle/models.py) on the neighbour-list oracle's edges: energies to 1e-6 eV,
    forces to 1e-5 eV/A."""
    import torch

    import md_oracle
    from oracle import models as om
    from oracle import nl as onl

    s = systems.perovskite(3, sigma=0.2)
    f_vec, e_vec = md_oracle.morse_forces(s)(s.positions)
    cell32 = s.cell.astype(np.float32)
    inv = np.linalg.inv(cell32.astype(np.float64)).astype(np.float32)
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    cand = onl.candidates(wrapped, cell32, np.float32(36.0 + 1e-3), 200)
    b = onl.build(s.positions, inv, cell32, cand, s.positions.astype(np.float32), wraps, np.float32(36.0),
                  np.float32(1.0), (1, 0, 0), int(cand.num_neighbors.sum()))
    e = b.n_edges
    energy, f, _ = om.energy_and_forces(
        om.morse_node_energy, torch.tensor(s.positions - wraps @ s.cell), torch.tensor(s.cell),
        torch.tensor(b.center[:e].astype(np.int64)), torch.tensor(b.neighbor[:e].astype(np.int64)),
        torch.tensor(b.images[:e]))
    assert abs(float(energy) - e_vec) < 1e-6
    assert np.abs(f.numpy() - f_vec).max() < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("when", ["construction", "growth"])
def test_auto_mode_falls_back_to_eager_on_out_of_memory(device, monkeypatch, when):
    """execution="auto" (gpu_md.py:1720-1774): an out-of-memory error injected from the host into a
    whole-step capture, at construction or at a capacity growth, continues the run on the eager
    path from the settled state; the trajectory equals a pure eager run bitwise. The same error
    in execution="whole_step" propagates."""
    import torch

    from fastmd_amd.execution import whole_step_cuda_graph as ws

    real_capture = ws.WholeStepGraphRunner._capture
    calls = {"capture": 0, "settle": 0}

    def capture(self):
        calls["capture"] += 1
        if when == "construction" or calls["capture"] == 2:
            raise torch.OutOfMemoryError("injected: HIP out of memory")
        return real_capture(self)

    real_settle = ws.WholeStepGraphRunner.settle

    def settle(self, stats):
        calls["settle"] += 1
        if when == "growth" and calls["settle"] == 2:
            # what an overflowed window's settle leaves: the window's start, then the overflow
            self.integrator.restore()
            raise ws.FixedCapacityOverflow(self.builder.e_capacity + 2, 0)
        return real_settle(self, stats)

    monkeypatch.setattr(ws.WholeStepGraphRunner, "_capture", capture)
    monkeypatch.setattr(ws.WholeStepGraphRunner, "settle", settle)
    with pytest.warns(RuntimeWarning, match="out of GPU memory"):
        md = _md(_adapter("morse", device), "auto", device, steps_per_launch=5)
        md.launch_behind = False
        md.run(30)
    assert md.execution == "eager" and md.whole_step_runner is None and md.steps == 30
    eager = _md(_adapter("morse", device), "eager", device)
    eager.run(30)
    torch.cuda.synchronize()
    assert torch.equal(_state(md), _state(eager))
    calls.update(capture=0, settle=0)
    with pytest.raises(torch.OutOfMemoryError):
        strict = _md(_adapter("morse", device), "whole_step", device, steps_per_launch=5)
        strict.launch_behind = False
        strict.run(30)
