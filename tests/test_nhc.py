"""(e) Nose-Hoover chain: the oracle pinned by invariants (CPU), the HIP kernels vs the oracle
(GPU, 1e-12 relative as the reference's ASE parity, tests/test_gpu_nhc.py:219-298)."""
import numpy as np
import pytest

from oracle import nhc as onhc
from fastmd_amd import systems, units


def _system(n_cells=2, seed=0, T=500.0):
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    s = systems.perovskite(n_cells, seed=seed)
    p = maxwell_boltzmann_momenta(s.masses, T, seed=0)
    return s, p


def test_units_match_ase_codata2014():
    assert units.kB == 8.617330337217213e-05
    assert units.fs == 0.09822694788464063
    assert onhc.KB == units.kB and abs(onhc.FS - units.fs) < 1e-17


def test_maxwell_boltzmann_is_numpy_default_rng():
    """ASE's MaxwellBoltzmannDistribution(rng=default_rng(0)): xi * sqrt(m kB T), bitwise."""
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    m = np.array([133.0, 119.0, 127.0])
    p = maxwell_boltzmann_momenta(m, 500.0, seed=0)
    xi = np.random.default_rng(0).standard_normal((3, 3))
    assert np.array_equal(p, xi * np.sqrt(m * units.kB * 500.0)[:, None])


def test_constants_layout_and_set_temperature_identity():
    from fastmd_amd.execution.gpu_nhc import nhc_constants

    c = nhc_constants(135, temperature_K=500.0, timestep=0.25 * units.fs, tdamp=25 * units.fs, tchain=3, tloop=1)
    assert len(c.values) == 16 + 2 * 3
    kT = units.kB * 500.0
    assert c.values[2] == kT and c.values[3] == 3 * 135 * kT
    assert c.values[16] == 3 * 135 * kT * (25 * units.fs) ** 2 and c.values[17] == kT * (25 * units.fs) ** 2
    w = c.values[4]
    assert w == (1 / (2 - 2 ** (1 / 3))) * (0.25 * units.fs / 2)
    assert c.values[5:8] == [w / 2, -(w / 4), -w]
    again = nhc_constants(135, temperature_K=500.0, timestep=0.25 * units.fs, tdamp=25 * units.fs, tchain=3, tloop=1)
    assert again.values == c.values


def _run_oracle(n_steps, dtype=np.float64, tchain=3, tloop=1, dt_fs=1.0, tdamp_fs=20.0, T=300.0, k=0.5):
    s, p = _system()
    f = onhc.harmonic(s.positions, k, dtype=dtype)
    f0, e0 = f(s.positions)
    o = onhc.NHC(s.masses, s.positions, p, temperature_K=T, timestep=dt_fs * units.fs, tdamp=tdamp_fs * units.fs,
                 tchain=tchain, tloop=tloop, f32_kick=dtype == np.float32, forces=f0, energy=e0)
    cons = [o.conserved_energy()]
    for _ in range(n_steps):
        o.step(f)
        cons.append(o.conserved_energy())
    return o, np.array(cons)


def test_oracle_conserves_extended_energy():
    """The NHC extended Hamiltonian is conserved to O(dt^2): a dropped term or a wrong sign in the
    chain (eta, p_eta, kT, Q) breaks this by orders of magnitude."""
    o, cons = _run_oracle(400)
    ekin_scale = o.kinetic_energy()
    assert np.max(np.abs(cons - cons[0])) < 1e-4 * ekin_scale
    # and the thermostat acted: the chain moved and exchanged energy
    assert np.abs(o.eta).max() > 1e-4 and np.abs(o.thermostat_energy()) > 1e-5 * ekin_scale


def test_oracle_time_reversible():
    """Velocity Verlet + symmetric Suzuki-Yoshida NHC is time reversible: run, flip p and p_eta,
    run again -> back to the start (the conserved-energy test does not see a chain-order error,
    this one does)."""
    s, p = _system()
    f = onhc.harmonic(s.positions + 0.05, 0.5)
    f0, e0 = f(s.positions)
    o = onhc.NHC(s.masses, s.positions, p, temperature_K=300.0, timestep=1.0 * units.fs, tdamp=20 * units.fs,
                 forces=f0, energy=e0)
    q0 = o.q.copy()
    for _ in range(50):
        o.step(f)
    o.p *= -1
    o.p_eta *= -1
    for _ in range(50):
        o.step(f)
    assert np.max(np.abs(o.q - q0)) < 1e-9


def test_oracle_canonical_temperature():
    """Harmonic crystal thermostatted at T: time-averaged kinetic temperature -> T (kT and Q
    enter here; a wrong degree-of-freedom count or kT shows as a biased mean)."""
    s, p = _system(T=400.0)
    f = onhc.harmonic(s.positions, 2.0)
    f0, e0 = f(s.positions)
    o = onhc.NHC(s.masses, s.positions, p, temperature_K=400.0, timestep=2.0 * units.fs, tdamp=20 * units.fs,
                 forces=f0, energy=e0)
    temps = []
    for k in range(3000):
        o.step(f)
        if k >= 1000:
            temps.append(2 * o.kinetic_energy() / (3 * s.n_atoms * units.kB))
    assert abs(np.mean(temps) - 400.0) < 20.0


@pytest.mark.gpu
@pytest.mark.parametrize("force_dtype", ["float64", "float32"])
@pytest.mark.parametrize("tchain,tloop", [(3, 1), (1, 1), (5, 2)])
def test_gpu_nhc_matches_oracle(device, force_dtype, tchain, tloop):
    import torch

    from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT

    print(f"[nhc] {force_dtype} tchain={tchain} tloop={tloop}", flush=True)
    dtype = np.float64 if force_dtype == "float64" else np.float32
    s, p = _system()
    f = onhc.harmonic(s.positions, 0.5, dtype=dtype)
    f0, e0 = f(s.positions)
    kw = dict(temperature_K=300.0, timestep=units.fs, tdamp=20 * units.fs, tchain=tchain, tloop=tloop)
    o = onhc.NHC(s.masses, s.positions, p, f32_kick=dtype == np.float32, forces=f0, energy=e0, **kw)
    g = GPUNoseHooverChainNVT(s.masses, s.positions, p, forces=f0, potential_energy=e0, device=device,
                              force_dtype=torch.float32 if dtype == np.float32 else torch.float64, **kw)
    q0 = torch.tensor(s.positions, device=device)
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    for _ in range(300):
        o.step(f)
        q = g.step_pre_force()
        d = q.to(tdt) - q0.to(tdt)
        fg = (-0.5 if dtype == np.float64 else torch.tensor(-0.5, dtype=tdt, device=device)) * d
        g.step_post_force(fg, energy=torch.tensor([o.e], device=device, dtype=torch.float64))
    st = g.state.numpy()
    for name, ref in (("positions", o.q), ("momenta", o.p), ("eta", o.eta), ("p_eta", o.p_eta)):
        rel = np.max(np.abs(st[name] - ref)) / max(np.max(np.abs(ref)), 1e-300)
        assert rel < 1e-12, (name, rel)
    cons = float(g.conserved_energy())
    assert abs(cons - o.conserved_energy()) < 1e-10 * abs(o.kinetic_energy())


@pytest.mark.gpu
@pytest.mark.parametrize("n_cells", [(8, 10, 10), (10, 10, 20)])
def test_gpu_nhc_large_systems(device, n_cells):
    """4 000 and 10 000 atoms: the register path at its limit and the streaming path (the chain
    run by the last workgroup to finish its partials): within 1e-12 of the oracle, and a second
    integrator over the same steps gives the same bits."""
    import torch

    from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT, maxwell_boltzmann_momenta

    print(f"[nhc-large] {n_cells}", flush=True)
    s = systems.perovskite(n_cells)
    p = maxwell_boltzmann_momenta(s.masses, 500.0, seed=0)
    f = onhc.harmonic(s.positions, 0.3)
    f0, e0 = f(s.positions)
    kw = dict(temperature_K=500.0, timestep=0.25 * units.fs, tdamp=25 * units.fs)
    o = onhc.NHC(s.masses, s.positions, p, forces=f0, energy=e0, **kw)
    g = GPUNoseHooverChainNVT(s.masses, s.positions, p, forces=f0, potential_energy=e0, device=device, **kw)
    g2 = GPUNoseHooverChainNVT(s.masses, s.positions, p, forces=f0, potential_energy=e0, device=device, **kw)
    q0 = torch.tensor(s.positions, device=device)
    for _ in range(20):
        o.step(f)
        for gi in (g, g2):
            q = gi.step_pre_force()
            gi.step_post_force(-0.3 * (q - q0), energy=torch.tensor([o.e], device=device, dtype=torch.float64))
    st = g.state.numpy()
    st2 = g2.state.numpy()
    for name in ("positions", "momenta", "eta", "p_eta"):
        assert np.array_equal(st[name], st2[name]), name
    for name, ref in (("positions", o.q), ("momenta", o.p), ("p_eta", o.p_eta)):
        rel = np.max(np.abs(st[name] - ref)) / np.max(np.abs(ref))
        assert rel < 1e-12, (name, rel)


@pytest.mark.gpu
@pytest.mark.parametrize("n_cells", [3, (8, 10, 10), (10, 10, 20)])
@pytest.mark.parametrize("force_dtype", ["float32", "float64"])
def test_gpu_nhc_post_pre_fused_bitwise(device, n_cells, force_dtype):
    """fmd_nhc_post_pre (step n's post-force half and step n + 1's pre-force half in one launch;
    three launches instead of four on the multi-block path) leaves the same state, bit for bit, as
    the two halves called one after the other: 135, 4 000 and 10 000 atoms, float32 and float64
    forces, with the energy copied; and the integration stays within 1e-12 of the oracle."""
    import torch

    from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT, maxwell_boltzmann_momenta

    print(f"[nhc-fused] {n_cells} {force_dtype}", flush=True)
    s = systems.perovskite(n_cells)
    p = maxwell_boltzmann_momenta(s.masses, 500.0, seed=0)
    f = onhc.harmonic(s.positions, 0.3)
    f0, e0 = f(s.positions)
    kw = dict(temperature_K=500.0, timestep=0.25 * units.fs, tdamp=25 * units.fs)
    o = onhc.NHC(s.masses, s.positions, p, forces=f0, energy=e0, **kw)
    sep = GPUNoseHooverChainNVT(s.masses, s.positions, p, forces=f0, potential_energy=e0, device=device, **kw)
    fus = GPUNoseHooverChainNVT(s.masses, s.positions, p, forces=f0, potential_energy=e0, device=device, **kw)
    q0 = torch.tensor(s.positions, device=device)
    dt = getattr(torch, force_dtype)
    q_f = fus.step_pre_force()
    steps = 12
    for k in range(steps):
        o.step(f)
        q_s = sep.step_pre_force()
        e = torch.tensor([o.e], device=device, dtype=torch.float64)
        sep.step_post_force((-0.3 * (q_s - q0)).to(dt), energy=e)
        forces = (-0.3 * (q_f - q0)).to(dt)
        if k + 1 < steps:
            q_f = fus.step_post_pre(forces, energy=e)
        else:
            fus.step_post_force(forces, energy=e)
        if k + 1 < steps:  # the fused integrator is half a step ahead: compare after its pre half
            sep_next = sep.state.numpy()
            fus_now = fus.state.numpy()
            assert np.array_equal(sep_next["forces"], fus_now["forces"])
    a, b = sep.state.numpy(), fus.state.numpy()
    for name in ("positions", "momenta", "forces", "eta", "p_eta", "potential_energy"):
        assert np.array_equal(a[name], b[name]), name
    if force_dtype == "float64":
        for name, ref in (("positions", o.q), ("momenta", o.p), ("p_eta", o.p_eta)):
            rel = np.max(np.abs(a[name] - ref)) / np.max(np.abs(ref))
            assert rel < 1e-12, (name, rel)


@pytest.mark.gpu
def test_gpu_nhc_set_temperature_and_rollback(device):
    import torch

    from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT

    s, p = _system()
    kw = dict(timestep=units.fs, tdamp=20 * units.fs)
    a = GPUNoseHooverChainNVT(s.masses, s.positions, p, temperature_K=300.0, device=device, **kw)
    a.set_temperature(450.0)
    b = GPUNoseHooverChainNVT(s.masses, s.positions, p, temperature_K=450.0, device=device, **kw)
    torch.cuda.synchronize()
    assert torch.equal(a.consts, b.consts)
    a.backup()
    before = a.state.flat.clone()
    a.step(lambda q: torch.zeros_like(q))
    assert not torch.equal(a.state.flat, before)
    a.restore()
    assert torch.equal(a.state.flat, before)
