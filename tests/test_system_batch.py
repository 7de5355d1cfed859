"""Heterogeneous multi-system batching (fastmd/execution/system_batch.py): systems with their own
atoms, cells and thermostats in slots of one whole-step graph; each system's trajectory equals its
single-system run bitwise and follows the CPU oracle's integration."""
import dataclasses

import numpy as np
import pytest

from fastmd_amd import systems
from fastmd_amd.config import InferenceConfig


def _sheared(s, shear):
    """``s`` in a sheared cell: the same fractional coordinates, cell rows plus ``shear``."""
    cell = s.cell + np.asarray(shear, dtype=np.float64)
    return systems.System((s.positions @ np.linalg.inv(s.cell)) @ cell, cell, s.numbers, s.masses)


def _systems():
    """Three systems of different sizes and cells: the cubic 135-atom perovskite, a 3 x 3 x 4
    (180 atoms, tetragonal) one and a sheared copy of a differently jittered 135-atom one."""
    return [systems.perovskite(3), systems.perovskite((3, 3, 4), seed=1),
            _sheared(systems.perovskite(3, seed=2), [[0, 0, 0], [0.8, 0, 0], [0.3, -0.5, 0]])]


def _adapter(name, device):
    if name == "morse":
        from fastmd_amd.models.pair_potential import MorsePairAdapter

        return MorsePairAdapter(device=device)
    if name == "mace_like":
        from fastmd_amd.models.mace_like import MaceLikeAdapter

        return MaceLikeAdapter(device=device)
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter, ThreeBodyConfig

    return ThreeBodyAdapter(config=ThreeBodyConfig(bond_cutoff=3.5), device=device)


def test_slot_layout_and_energy_ranges():
    from fastmd_amd.engine.energy_derivative import _ranges
    from fastmd_amd.execution.system_batch import SlotLayout

    layout = SlotLayout((140, 180, 150))
    assert layout.starts == (0, 140, 320) and layout.rows == 470 and layout.count == 3
    assert _ranges(3, 12) == [(0, 4), (4, 4), (8, 4)]
    assert _ranges(((0, 135), (140, 180)), 470) == [(0, 135), (140, 180)]
    with pytest.raises(ValueError):
        _ranges(((400, 100),), 470)
    with pytest.raises(ValueError):
        SlotLayout((10, 0))


def _single(s, adapter, momenta, device, steps):
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics

    md = GPUResidentMolecularDynamics(s, model=adapter, device=device, temperature=500.0, timestep=0.25,
                                      tdamp=25.0, momenta=momenta, steps_per_launch=5,
                                      config=InferenceConfig(execution="whole_step"))
    md.run(steps)
    return md


@pytest.mark.gpu
@pytest.mark.parametrize("model_name", ["morse", "mace_like", "threebody"])
def test_systems_equal_single_runs_bitwise(device, model_name):
    """Three different systems (135 / 180 / 135 atoms, cubic / tetragonal / sheared cells), two slots
    with vacant rows: after 30 steps every system's positions, momenta, forces, energy and chain
    equal its single-system run bitwise."""
    import torch

    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.execution.system_batch import SystemBatchedMD

    print(f"[systems] {model_name}", flush=True)
    sys_list = _systems()
    momenta = [maxwell_boltzmann_momenta(s.masses, 500.0, 20 + k) for k, s in enumerate(sys_list)]
    batch = SystemBatchedMD(sys_list, _adapter(model_name, device), ceilings=(140, 180, 150), device=device,
                            temperature=500.0, timestep=0.25, tdamp=25.0, momenta=momenta, steps_per_launch=5)
    batch.run(30)
    torch.cuda.synchronize()
    assert batch.runner.builder.batch.systems.count == 3
    for k, s in enumerate(sys_list):
        single = _single(s, _adapter(model_name, device), momenta[k], device, 30)
        torch.cuda.synchronize()
        got = batch.system_state(k)
        th = single.integrator
        for key in ("positions", "momenta", "forces"):
            assert torch.equal(got[key], getattr(th, key)), (k, key)
        assert torch.equal(got["potential_energy"].reshape(1), th.potential_energy.reshape(1)), k
        assert torch.equal(batch.integrator.eta[k], th.eta) and torch.equal(batch.integrator.p_eta[k], th.p_eta)
    vacant = batch.integrator.state.positions[135:140]
    assert torch.count_nonzero(vacant) == 0  # vacant rows stay parked
    thermo = batch.thermodynamics()
    assert [t["atoms"] for t in thermo] == [135, 180, 135]


@pytest.mark.gpu
def test_small_and_large_systems_against_single_runs(device):
    """A 135-atom system in a slot of 2 200 rows next to the 5 000-atom perovskite, 10 steps. The
    message kernels take the small system's atoms four waves each and the large one's one wave
    each, as their single runs do (chosen per system, not per slot or union), and the large
    system's chain runs on the multi-block NHC path (more than 4 096 atoms): the large system
    equals its single run bitwise. The small system's node GEMMs run inside launches of the
    union's 7 200 rows, which take the split-plane form its 135-atom single run does not (the
    form is chosen per launch size), so it matches its single run to float32 rounding, not
    bitwise."""
    import torch

    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.execution.system_batch import SystemBatchedMD
    from fastmd_amd.models.mace_like import SPLIT_ROWS_MAX_ATOMS

    print("[systems] 135 + 5000 atoms, mace_like", flush=True)
    sys_list = [systems.perovskite(3), systems.perovskite(10, seed=3)]
    assert sys_list[0].n_atoms <= SPLIT_ROWS_MAX_ATOMS < 2200 < sys_list[1].n_atoms
    momenta = [maxwell_boltzmann_momenta(s.masses, 500.0, 40 + k) for k, s in enumerate(sys_list)]
    batch = SystemBatchedMD(sys_list, _adapter("mace_like", device), ceilings=(2200, 5000), device=device,
                            temperature=500.0, timestep=0.25, tdamp=25.0, momenta=momenta, steps_per_launch=5)
    assert batch.runner.builder.batch.system_slots == ((0, 2200, 135), (2200, 5000, 5000))
    batch.run(10)
    torch.cuda.synchronize()
    for k, s in enumerate(sys_list):
        single = _single(s, _adapter("mace_like", device), momenta[k], device, 10)
        torch.cuda.synchronize()
        got = batch.system_state(k)
        th = single.integrator
        if k == 1:
            for key in ("positions", "momenta", "forces"):
                assert torch.equal(got[key], getattr(th, key)), (k, key)
            assert torch.equal(got["potential_energy"].reshape(1), th.potential_energy.reshape(1))
            assert torch.equal(batch.integrator.eta[k], th.eta) and torch.equal(batch.integrator.p_eta[k], th.p_eta)
        else:
            dq = float((got["positions"] - th.positions).abs().max())
            df = float((got["forces"] - th.forces).abs().max())
            de = abs(float(got["potential_energy"]) - float(th.potential_energy)) / s.n_atoms
            print(f"[systems] 135-atom system vs its single run: |dq| {dq:.2e} A, |dF| {df:.2e} eV/A, "
                  f"|dE| {de:.2e} eV/atom", flush=True)
            assert dq < 1e-6 and df < 1e-4 and de < 1e-6
        del single
        torch.cuda.empty_cache()


def test_wave_groups_follow_each_systems_size():
    """The message kernels' launches of a slot union: one per run of slots with the same waves per
    atom, over that run's range of the atom order."""
    import types

    import torch

    from fastmd_amd.models.mace_like import _wave_groups

    order = torch.arange(7400, dtype=torch.int32)
    base = order.data_ptr()
    batch = types.SimpleNamespace(atom_order=order, max_system_rows=5000,
                                  system_slots=((0, 2200, 135), (2200, 5000, 5000), (7200, 200, 180)))
    assert _wave_groups(batch, 7400) == [(base, 2200, 4), (base + 4 * 2200, 5000, 1), (base + 4 * 7200, 200, 4)]
    batch.system_slots = ((0, 2200, 135), (2200, 200, 180), (2400, 5000, 5000))
    assert _wave_groups(batch, 7400) == [(base, 2400, 4), (base + 4 * 2400, 5000, 1)]
    single = types.SimpleNamespace(atom_order=None, max_system_rows=0)
    assert _wave_groups(single, 135) == [(None, 135, 4)] and _wave_groups(single, 3000) == [(None, 3000, 1)]
    replicas = types.SimpleNamespace(atom_order=None, max_system_rows=135)
    assert _wave_groups(replicas, 135 * 32) == [(None, 135 * 32, 4)]


@pytest.mark.gpu
@pytest.mark.parametrize("model_name", ["morse", "mace_like"])
def test_systems_follow_the_oracle_md(device, model_name):
    """Each system of the union follows the CPU oracle's NHC integration of that system alone
    (tests/md_oracle.py): positions to 1e-4 A and the conserved quantity's change since step 0 to
    1e-6 eV per atom, at every 10th of 50 steps."""
    import md_oracle
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.execution.system_batch import SystemBatchedMD

    sys_list = _systems()
    momenta = [maxwell_boltzmann_momenta(s.masses, 500.0, 30 + k) for k, s in enumerate(sys_list)]
    if model_name == "morse":
        forces = [md_oracle.morse_forces(s) for s in sys_list]
    else:
        from fastmd_amd.models.mace_like import MaceLike, MaceLikeConfig

        params = {k: v.detach().clone() for k, v in MaceLike(MaceLikeConfig()).named_parameters()}
        forces = [md_oracle.mace_like_forces(s, params, dataclasses.asdict(MaceLikeConfig())) for s in sys_list]
    batch = SystemBatchedMD(sys_list, _adapter(model_name, device), ceilings=(140, 180, 150), device=device,
                            temperature=500.0, timestep=0.25, tdamp=25.0, momenta=momenta, steps_per_launch=5)
    oracles = [md_oracle.run_nhc(s, f, p, 50, sample_every=10, positions_until=50)
               for s, f, p in zip(sys_list, forces, momenta)]
    c0 = [t["conserved_energy"] for t in batch.thermodynamics()]
    for k in range(1, 6):
        batch.run(10)
        thermo = batch.thermodynamics()
        for s_idx, (s, o) in enumerate(zip(sys_list, oracles)):
            q = batch.system_state(s_idx)["positions"].cpu().numpy()
            dq = float(np.abs(q - o["positions"][k]).max())
            dc = abs((thermo[s_idx]["conserved_energy"] - c0[s_idx]) - (o["conserved"][k] - o["conserved"][0]))
            assert dq < 1e-4, (s_idx, k, dq)
            assert dc < 1e-6 * s.n_atoms, (s_idx, k, dc)
    print(f"[systems vs oracle] {model_name}: 50 steps ok", flush=True)


@pytest.mark.gpu
def test_write_system_swaps_a_slot(device):
    """After 20 steps, another system (150 atoms of a 3 x 2 x 5 supercell) is written into the
    180-row slot: it then runs bitwise as its own single-system run, and the other systems
    continue bitwise as theirs."""
    import torch

    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.execution.system_batch import SystemBatchedMD

    sys_list = _systems()
    momenta = [maxwell_boltzmann_momenta(s.masses, 500.0, 40 + k) for k, s in enumerate(sys_list)]
    batch = SystemBatchedMD(sys_list, _adapter("morse", device), ceilings=(140, 180, 150), device=device,
                            temperature=500.0, timestep=0.25, tdamp=25.0, momenta=momenta, steps_per_launch=5)
    batch.run(20)
    new = systems.perovskite((3, 2, 5), seed=5)
    p_new = maxwell_boltzmann_momenta(new.masses, 500.0, 99)
    batch.write_system(1, new, momenta=p_new)
    batch.run(20)
    torch.cuda.synchronize()
    assert batch.thermodynamics()[1]["atoms"] == 150
    expected = [(sys_list[0], momenta[0], 40), (new, p_new, 20), (sys_list[2], momenta[2], 40)]
    for k, (s, p, steps) in enumerate(expected):
        single = _single(s, _adapter("morse", device), p, device, steps)
        torch.cuda.synchronize()
        got = batch.system_state(k)
        for key in ("positions", "momenta", "forces"):
            assert torch.equal(got[key], getattr(single.integrator, key)), (k, key)
    with pytest.raises(ValueError):
        batch.write_system(0, systems.perovskite((3, 3, 4)))  # 180 atoms > the 140-row slot


@pytest.mark.gpu
def test_reference_entry_point_runs_the_union(device):
    """MultiSystemMolecularDynamics(model, systems, ...) with the reference's argument names: the
    momenta of seed + s, slot_atoms as one ceiling for every slot; equal to SystemBatchedMD."""
    import torch

    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.execution.system_batch import SystemBatchedMD
    from fastmd_amd.interfaces.multi_system_md import MultiSystemMolecularDynamics

    sys_list = _systems()
    md = MultiSystemMolecularDynamics(_adapter("morse", device), sys_list, temperature=500.0, timestep=0.25,
                                      taut=25.0, seed=7, steps_per_launch=5, slot_atoms=180, device=device)
    assert md.layout.ceilings == (180, 180, 180)
    momenta = [maxwell_boltzmann_momenta(s.masses, 500.0, 7 + k) for k, s in enumerate(sys_list)]
    ref = SystemBatchedMD(sys_list, _adapter("morse", device), ceilings=(180, 180, 180), device=device,
                          temperature=500.0, timestep=0.25, tdamp=25.0, momenta=momenta, steps_per_launch=5)
    md.run(10)
    ref.run(10)
    torch.cuda.synchronize()
    for k in range(3):
        assert torch.equal(md.system_state(k)["positions"], ref.system_state(k)["positions"])
    with pytest.raises(NotImplementedError):
        MultiSystemMolecularDynamics(_adapter("morse", device), sys_list, ensemble="nve", device=device)
