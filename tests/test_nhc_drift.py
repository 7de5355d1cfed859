"""The north-star drift gate: the NHC conserved quantity of the GPU's whole-step MD drifts no more
than the CPU oracle's integration of the same system.

The oracle's integrations (``tests/golden/make_nhc_drift.py``) are committed fixtures: 10 000
Morse steps and 2 000 MACE-like steps, each from the momenta of seeds
0, 1 and 2. The CPU tests pin each fixture to a short live run of the oracle. The trajectories of
two chaotic runs decorrelate within a few hundred steps, so over the whole run the size of the
drift is compared, not the path.

Drift is the systematic change of C(t) over the run: the least-squares slope of the sampled C(t)
times the run length, |b| * T. The largest excursion max_t |C(t) - C(0)| is not used as the
gate: with a float32 model it is about four standard deviations of the energy's rounding noise
(about 2e-6 eV at 135 atoms, five times the fitted drift of the float32 oracle over 2 000 steps)
and so compares noise amplitudes, not drift. The gate is

    mean over seeds (GPU |b| T) <= mean over seeds (oracle |b| T) + (max - min of the oracle's |b| T)

i.e. the oracle's own spread across momenta seeds is the noise floor. The excursion and the
residual standard deviation about the fitted line are reported beside it. Over the first steps,
while the paths still agree, the positions themselves are compared.
"""
import os

import numpy as np
import pytest

from fastmd_amd import systems

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _fixture(name):
    return np.load(os.path.join(GOLDEN, name))


def drift_stats(steps, conserved):
    """(|b| T, residual std, max |C - C0|) of one sampled C(t) series: b is the least-squares slope
    in eV per step, T the number of steps from the first to the last sample."""
    t = np.asarray(steps, dtype=np.float64)
    c = np.asarray(conserved, dtype=np.float64) - float(conserved[0])
    design = np.stack([np.ones_like(t), t], axis=1)
    coef = np.linalg.lstsq(design, c, rcond=None)[0]
    resid = c - design @ coef
    return abs(float(coef[1])) * float(t[-1] - t[0]), float(resid.std()), float(np.abs(c).max())


def _gate(gpu, oracle):
    gpu, oracle = np.asarray(gpu), np.asarray(oracle)
    return float(gpu.mean()), float(oracle.mean() + (oracle.max() - oracle.min()))


def _record(name, rows, directory):
    """Prints the per-seed drift figures of one gate (run pytest with -s to see them) and writes
    them to ``directory`` (the test's tmp_path)."""
    lines = ["seed run drift_|b|T_eV resid_std_eV max_excursion_eV"]
    lines += [" ".join(str(v) for v in row) for row in rows]
    with open(os.path.join(directory, f"drift_{name}.txt"), "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print(f"[drift {name}]\n" + "\n".join(lines), flush=True)


def _mace_params():
    import dataclasses

    from fastmd_amd.models.mace_like import MaceLike, MaceLikeConfig

    cfg = MaceLikeConfig()
    return {k: v.detach().clone() for k, v in MaceLike(cfg).named_parameters()}, dataclasses.asdict(cfg)


# ------------------------------------------------------------------------------------ CPU pins
def test_morse_fixture_is_the_oracle_integration():
    import md_oracle
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    fx = _fixture("nhc_drift_morse_135.npz")
    s = systems.perovskite(3)
    assert tuple(fx["seeds"]) == (0, 1, 2) and fx["steps"][-1] == 10_000 and fx["conserved"].shape == (3, 101)
    live = md_oracle.run_nhc(s, md_oracle.morse_forces(s), maxwell_boltzmann_momenta(s.masses, 500.0, 1), 300,
                             sample_every=100)
    np.testing.assert_allclose(live["conserved"], fx["conserved"][1, :4], rtol=0, atol=1e-9)


def test_mace_like_fixture_is_the_oracle_integration():
    import torch

    import md_oracle
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    fx = _fixture("nhc_drift_mace_like_135.npz")
    s = systems.perovskite(3)
    assert fx["conserved_f64"].shape == (3, 201) and fx["conserved_f32"].shape == (3, 201)
    assert fx["positions_f64"].shape == (3, 6, s.n_atoms, 3)
    params, cfg = _mace_params()
    p0 = maxwell_boltzmann_momenta(s.masses, 500.0, 0)
    for dtype, key in ((torch.float64, "conserved_f64"), (torch.float32, "conserved_f32")):
        live = md_oracle.run_nhc(s, md_oracle.mace_like_forces(s, params, cfg, dtype=dtype), p0, 20,
                                 positions_until=20)
        np.testing.assert_allclose(live["conserved"], fx[key][0, :3], rtol=0, atol=1e-9)
        if dtype == torch.float64:
            np.testing.assert_allclose(live["positions"], fx["positions_f64"][0, :3], rtol=0, atol=1e-10)
    # the oracle's float32 and float64 paths are the same trajectory to float32 noise early on
    assert np.abs(fx["conserved_f32"][:, :6] - fx["conserved_f64"][:, :6]).max() < 1e-3


def test_drift_stats_separates_trend_from_noise():
    """A planted linear trend of 1e-6 eV over 2 000 steps under 2e-6 eV of white noise is recovered
    by the fitted |b| T to within its standard error, while the excursion is set by the noise."""
    t = np.arange(201) * 10.0
    noise = np.random.default_rng(0).normal(0.0, 2e-6, t.shape)
    drift, resid, excursion = drift_stats(t, -5.0 + 5e-10 * t + noise)
    se = 2e-6 * np.sqrt(12.0 / t.size)  # standard error of |b| T for white noise
    assert abs(drift - 1e-6) < 3 * se
    assert 1.8e-6 < resid < 2.2e-6 and excursion > 3 * drift
    assert drift_stats(t, 2.0 - 1e-7 * t)[0] == pytest.approx(2e-4, rel=1e-12)


def test_oracle_pair_list_matches_the_neighbour_list_oracle():
    """The fixtures' brute-force skin pair list holds exactly the neighbour-list oracle's edges
    (away from the cutoff) on a jittered, displaced system."""
    import md_oracle
    from oracle import nl as onl

    s = systems.perovskite(3, sigma=0.2)
    q = s.positions + np.random.default_rng(3).normal(0, 0.3, s.positions.shape)
    ii, jj, img = md_oracle.PairList(s.cell).pairs(q)
    cell32 = s.cell.astype(np.float32)
    inv = np.linalg.inv(cell32.astype(np.float64)).astype(np.float32)
    _, wraps, wrapped = onl.wrap(q, inv, cell32)
    cand = onl.candidates(wrapped, cell32, np.float32(64.0), 1504)
    b = onl.build(q, inv, cell32, cand, q.astype(np.float32), wraps, np.float32(36.0), np.float32(2.0), (1, 0, 0),
                  10 ** 6)
    e = b.n_edges
    # the builder's images are in the frame of the wrapped positions: move them to q's frame
    w = wraps.astype(np.int64)
    nl_img = b.images[:e].astype(np.int64) - w[b.neighbor[:e]] + w[b.center[:e]]
    ours = {(int(i), int(j), *map(int, k)) for i, j, k in zip(ii, jj, img)}
    theirs = {(int(i), int(j), *map(int, k)) for i, j, k in zip(b.center[:e], b.neighbor[:e], nl_img)}
    vec = lambda i, j, k: q[j] + np.asarray(k) @ s.cell - q[i]  # noqa: E731
    near = {t for t in ours ^ theirs if abs(np.linalg.norm(vec(t[0], t[1], t[2:])) - 6.0) < 1e-5}
    assert ours ^ theirs == near and len(ours) > 1000


# ------------------------------------------------------------------------------------ GPU gates
def _md(system, adapter, momenta, device):
    from fastmd_amd.config import InferenceConfig
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics

    return GPUResidentMolecularDynamics(system, model=adapter, device=device, temperature=500.0, timestep=0.25,
                                        tdamp=25.0, momenta=momenta, steps_per_launch=10,
                                        config=InferenceConfig(execution="whole_step"))


@pytest.mark.gpu
def test_nhc_conserved_quantity_drift_10k_steps_morse(device, tmp_path):
    """10 000 whole-step NHC steps of Morse on the 135-atom perovskite at 500 K."""
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.models.pair_potential import MorsePairAdapter

    fx = _fixture("nhc_drift_morse_135.npz")
    s = systems.perovskite(3)
    gpu, oracle, rows = [], [], []
    for k, seed in enumerate(fx["seeds"]):
        md = _md(s, MorsePairAdapter(device=device), maxwell_boltzmann_momenta(s.masses, 500.0, int(seed)), device)
        c0 = md.conserved_energy()
        assert abs(c0 - fx["conserved"][k, 0]) < 1e-6 * s.n_atoms
        series = [c0]
        for _ in range(100):
            md.run(100)
            series.append(md.conserved_energy())
        g, o = drift_stats(fx["steps"], series), drift_stats(fx["steps"], fx["conserved"][k])
        gpu.append(g[0])
        oracle.append(o[0])
        rows += [(int(seed), "gpu", *g), (int(seed), "oracle", *o)]
        print(f"[drift morse] seed {seed}: |b|T gpu {g[0]:.3e} eV, oracle {o[0]:.3e} eV; "
              f"residual std gpu {g[1]:.3e}, oracle {o[1]:.3e}; excursion gpu {g[2]:.3e}, oracle {o[2]:.3e}",
              flush=True)
    _record("morse_135_10000", rows, tmp_path)
    got, bound = _gate(gpu, oracle)
    print(f"[drift morse] mean gpu {got:.3e} eV <= bound {bound:.3e} eV", flush=True)
    assert got <= bound, (gpu, oracle)


@pytest.mark.gpu
def test_mace_like_nhc_2000_steps_vs_oracle(device, tmp_path):
    """the MACE-like model (random init, seed 0) on the 135-atom perovskite, 2 000
    whole-step NHC steps per seed. Positions follow the float64 oracle's trajectory over the first
    50 steps (1e-4 A); the drift over the whole run is gated against the oracle's float32 runs (the
    reference's arithmetic class; the float64 runs are reported beside them)."""
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.models.mace_like import MaceLikeAdapter

    fx = _fixture("nhc_drift_mace_like_135.npz")
    s = systems.perovskite(3)
    gpu, o32, rows = [], [], []
    for k, seed in enumerate(fx["seeds"]):
        md = _md(s, MaceLikeAdapter(device=device), maxwell_boltzmann_momenta(s.masses, 500.0, int(seed)), device)
        c0 = md.conserved_energy()
        assert abs(c0 - fx["conserved_f64"][k, 0]) < 1e-5 * s.n_atoms
        series, dev = [c0], [0.0]
        for block in range(200):
            md.run(10)
            series.append(md.conserved_energy())
            if block < 5:
                dev.append(float(np.abs(md.positions.cpu().numpy() - fx["positions_f64"][k, block + 1]).max()))
        print(f"[mace 2000] seed {seed}: max |dq| over 50 steps {max(dev):.2e} A", flush=True)
        assert max(dev) < 1e-4, dev
        g = drift_stats(fx["steps"], series)
        f32 = drift_stats(fx["steps"], fx["conserved_f32"][k])
        f64 = drift_stats(fx["steps"], fx["conserved_f64"][k])
        gpu.append(g[0])
        o32.append(f32[0])
        rows += [(int(seed), "gpu", *g), (int(seed), "oracle_f32", *f32), (int(seed), "oracle_f64", *f64)]
        print(f"[mace 2000] seed {seed}: |b|T gpu {g[0]:.3e} eV, oracle f32 {f32[0]:.3e} eV, oracle f64 "
              f"{f64[0]:.3e} eV; residual std gpu {g[1]:.3e}, oracle f32 {f32[1]:.3e}; excursion gpu "
              f"{g[2]:.3e}, oracle f32 {f32[2]:.3e}", flush=True)
    _record("mace_like_135_2000", rows, tmp_path)
    got, bound = _gate(gpu, o32)
    print(f"[mace 2000] mean gpu {got:.3e} eV <= bound {bound:.3e} eV", flush=True)
    assert got <= bound, (gpu, o32)


_LONG = os.path.join(GOLDEN, "nhc_drift_mace_like_135_10k.npz")
_needs_long = pytest.mark.skipif(not os.path.exists(_LONG), reason="tests/golden/make_nhc_drift.py mace_like_10k "
                                 "has not written its fixture")


@_needs_long
def test_mace_like_10k_fixture_is_the_oracle_integration():
    import torch

    import md_oracle
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    fx = _fixture("nhc_drift_mace_like_135_10k.npz")
    s = systems.perovskite(3)
    assert tuple(fx["seeds"]) == (0, 1, 2) and fx["steps"][-1] == 10_000
    assert fx["conserved_f32"].shape == (3, 201) and fx["conserved_f64"].shape == (3, 201)
    params, cfg = _mace_params()
    threads = torch.get_num_threads()
    torch.set_num_threads(1)  # the generator's workers run one thread each (float32 sums follow the thread count)
    try:
        live = md_oracle.run_nhc(s, md_oracle.mace_like_forces(s, params, cfg, dtype=torch.float32),
                                 maxwell_boltzmann_momenta(s.masses, 500.0, 2), 100, sample_every=50)
    finally:
        torch.set_num_threads(threads)
    np.testing.assert_allclose(live["conserved"], fx["conserved_f32"][2, :3], rtol=0, atol=1e-9)
    # the 2 000-step fixture is the same integration, sampled more often
    short = _fixture("nhc_drift_mace_like_135.npz")
    np.testing.assert_allclose(fx["conserved_f64"][:, :41], short["conserved_f64"][:, ::5], rtol=0, atol=1e-9)


@pytest.mark.gpu
@_needs_long
def test_mace_like_nhc_drift_10k_steps(device, tmp_path):
    """The north-star drift gate on configs[2]: 10 000 whole-step NHC steps of the MACE-like model
    (random init, seed 0) on the 135-atom perovskite per momenta seed, C(t) every 50 steps, the
    fitted drift gated against the oracle's float32 runs of the same 10 000 steps (float64 runs
    reported beside them)."""
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.models.mace_like import MaceLikeAdapter

    fx = _fixture("nhc_drift_mace_like_135_10k.npz")
    s = systems.perovskite(3)
    gpu, o32, rows = [], [], []
    for k, seed in enumerate(fx["seeds"]):
        md = _md(s, MaceLikeAdapter(device=device), maxwell_boltzmann_momenta(s.masses, 500.0, int(seed)), device)
        c0 = md.conserved_energy()
        assert abs(c0 - fx["conserved_f64"][k, 0]) < 1e-5 * s.n_atoms
        series = [c0]
        for _ in range(200):
            md.run(50)
            series.append(md.conserved_energy())
        g = drift_stats(fx["steps"], series)
        f32 = drift_stats(fx["steps"], fx["conserved_f32"][k])
        f64 = drift_stats(fx["steps"], fx["conserved_f64"][k])
        gpu.append(g[0])
        o32.append(f32[0])
        rows += [(int(seed), "gpu", *g), (int(seed), "oracle_f32", *f32), (int(seed), "oracle_f64", *f64)]
        print(f"[mace 10k] seed {seed}: |b|T gpu {g[0]:.3e} eV, oracle f32 {f32[0]:.3e} eV, oracle f64 "
              f"{f64[0]:.3e} eV; residual std gpu {g[1]:.3e}, oracle f32 {f32[1]:.3e}; excursion gpu "
              f"{g[2]:.3e}, oracle f32 {f32[2]:.3e}", flush=True)
    _record("mace_like_135_10000", rows, tmp_path)
    got, bound = _gate(gpu, o32)
    print(f"[mace 10k] mean gpu {got:.3e} eV <= bound {bound:.3e} eV", flush=True)
    assert got <= bound, (gpu, o32)
