"""Trajectory, thermo and restart outputs (fastmd/execution/gpu_logging.py, md_protocol.py): the
formats round-trip on the CPU; on the GPU a whole-step run writes its frames, thermo lines and
restart files, and a run resumed from a restart file continues the uninterrupted trajectory
bitwise."""
import io

import numpy as np
import pytest
import torch

from fastmd_amd import systems
from fastmd_amd.config import InferenceConfig
from fastmd_amd.execution import md_protocol as mp
from fastmd_amd.execution.gpu_logging import AsyncGPUMDLogger, AtomsTemplate, Frame


def _frame(rng, n=5, step=10):
    return Frame(numbers=np.array([55, 50, 53, 53, 53])[:n], masses=np.array([133.0, 119.0, 127.0, 127.0, 127.0])[:n],
                 cell=np.diag([6.2, 6.2, 6.3]), pbc=np.ones(3, bool), positions=rng.normal(size=(n, 3)),
                 momenta=rng.normal(size=(n, 3)), forces=rng.normal(size=(n, 3)), energy=-12.5,
                 info={"step": np.array([step]), "time_fs": np.array([2.5]), "nhc_eta": np.array([0.1, 0.2, 0.3])})


def test_extxyz_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    frames = [_frame(rng, step=10), _frame(rng, step=20)]
    traj = mp.ExtxyzTrajectory(tmp_path / "t.extxyz", append=False)
    for f in frames:
        traj.write(f)
    traj.close()
    back = mp.read_extxyz(tmp_path / "t.extxyz")
    assert len(back) == 2
    for f, b in zip(frames, back):
        assert b["symbols"] == ["Cs", "Sn", "I", "I", "I"]
        assert np.allclose(b["positions"], f.positions, atol=1e-8)
        assert np.allclose(b["velocities"], f.momenta / f.masses[:, None], atol=1e-8)
        assert np.allclose(b["forces"], f.forces, atol=1e-8)
        assert np.array_equal(b["cell"], f.cell) and b["pbc"].all() and b["energy"] == -12.5
        assert b["info"]["step"] == int(f.info["step"][0]) and isinstance(b["info"]["step"], int)
        assert np.array_equal(b["info"]["nhc_eta"], [0.1, 0.2, 0.3]) and b["info"]["time_fs"] == 2.5
    # append mode continues the file
    traj = mp.ExtxyzTrajectory(tmp_path / "t.extxyz", append=True)
    traj.write(frames[0])
    traj.close()
    assert len(mp.read_extxyz(tmp_path / "t.extxyz")) == 3


def test_extxyz_frame_text_is_the_ase_layout(tmp_path):
    """A written frame, character for character, as ASE's extxyz writer lays out an Atoms with
    explicit masses, velocities, a single-point calculator (energy, forces) and info entries:
    Lattice, Properties, the info keys in insertion order, energy, pbc; ``%-2s`` species and
    ``%16.8f`` columns (hand-written expected text)."""
    frame = Frame(numbers=np.array([55, 53]), masses=np.array([2.0, 4.0]), cell=np.diag([6.2, 6.2, 6.3]),
                  pbc=np.ones(3, bool), positions=np.array([[0.1, 0.2, 0.3], [3.1, 3.1, 0.0]]),
                  momenta=np.array([[2.0, -4.0, 0.0], [4.0, 0.0, -2.0]]),
                  forces=np.array([[0.5, -0.25, 0.0], [-0.5, 0.25, 1e-9]]), energy=-12.5,
                  info={"step": np.array([10.0]), "time_fs": np.array([2.5]), "nhc_eta": np.array([0.1, 0.2, 0.3])},
                  explicit_masses=True)
    traj = mp.ExtxyzTrajectory(tmp_path / "one.extxyz", append=False)
    traj.write(frame)
    traj.close()
    expected = (
        "2\n"
        'Lattice="6.2 0.0 0.0 0.0 6.2 0.0 0.0 0.0 6.3" '
        "Properties=species:S:1:pos:R:3:masses:R:1:velocities:R:3:forces:R:3 "
        'step=10 time_fs=2.5 nhc_eta="0.1 0.2 0.3" energy=-12.5 pbc="T T T"\n'
        "Cs       0.10000000       0.20000000       0.30000000       2.00000000       1.00000000"
        "      -2.00000000       0.00000000       0.50000000      -0.25000000       0.00000000\n"
        "I        3.10000000       3.10000000       0.00000000       4.00000000       1.00000000"
        "       0.00000000      -0.50000000      -0.50000000       0.25000000       0.00000000\n")
    assert (tmp_path / "one.extxyz").read_text() == expected
    back = mp.read_extxyz(tmp_path / "one.extxyz")[0]
    assert back["keys"] == ["Lattice", "Properties", "step", "time_fs", "nhc_eta", "energy", "pbc"]
    assert np.array_equal(back["masses"], [2.0, 4.0]) and np.allclose(back["velocities"], [[1, -2, 0], [1, 0, -0.5]])


def test_restart_round_trip_and_format_check(tmp_path):
    rng = np.random.default_rng(1)
    data = mp.RestartData(ids=np.arange(4), numbers=np.array([55, 50, 53, 53]), masses=rng.random(4),
                          positions=rng.normal(size=(4, 3)), momenta=rng.normal(size=(4, 3)),
                          forces=rng.normal(size=(4, 3)), energy=np.array(-3.0), reference_energy=np.array(-1.0),
                          cell=np.eye(3) * 6.2, pbc=np.ones(3, bool), step=120,
                          parameters={"ensemble": "nvt_nhc", "tchain": 3, "total_steps": 200},
                          temperature_K=500.0, nhc_state={"temperature_K": 500.0, "eta": np.arange(3.0),
                                                          "p_eta": -np.arange(3.0)},
                          offsets={mp.THERMO_FILE: 120, mp.TRAJECTORY_FILE: 4096}, engine="native")
    mp.write_restart(tmp_path / mp.RESTART_FILE, data)
    back = mp.read_restart(tmp_path / mp.RESTART_FILE)
    for key in ("ids", "numbers", "masses", "positions", "momenta", "forces", "cell", "pbc"):
        assert np.array_equal(getattr(back, key), getattr(data, key)), key
    assert back.step == 120 and back.temperature_K == 500.0 and back.engine == "native"
    assert back.parameters == data.parameters and back.offsets == data.offsets
    assert np.array_equal(back.nhc_state["eta"], np.arange(3.0)) and np.array_equal(back.nhc_state["p_eta"], -np.arange(3.0))
    np.savez(tmp_path / "other.npz", format=np.array("something/1"))
    with pytest.raises(ValueError, match="restart file"):
        mp.read_restart(tmp_path / "other.npz")
    assert mp.resume_mismatch({"a": 1, "total_steps": 5, "b": 2}, {"a": 1, "total_steps": 9, "b": 3}) == {"b": (2, 3)}


class _Failing:
    def write(self, frame):
        raise OSError("disk full")

    def close(self):
        pass


def test_logger_cpu_path_text_log_and_failure():
    """The logger on a CPU device (synchronous copies): the reference's text-log header and
    columns; a failing trajectory writer surfaces in the caller's thread."""
    n = 5
    tmpl = AtomsTemplate(np.array([55, 50, 53, 53, 53]), np.full(n, 127.0), np.eye(3) * 6.2, np.ones(3, bool))
    log = io.StringIO()
    lg = AsyncGPUMDLogger(tmpl, torch.device("cpu"), logfile=log, loginterval=10, state_dtype=torch.float64)
    assert lg.should_log(20) and not lg.should_log(15)
    z = torch.zeros(n, 3, dtype=torch.float64)
    for k in range(3):
        lg.enqueue(step=10 * k, time_ps=0.0025 * k, positions=z, momenta=z, forces=z.float(), cell=torch.eye(3),
                   potential_energy=torch.tensor(-1.5 - k), kinetic_energy=torch.tensor(0.25),
                   temperature=torch.tensor(300.0))
    lg.close()
    lines = log.getvalue().splitlines()
    assert lines[0] == "%-9s %12s %12s %12s  %6s" % ("Time[ps]", "Etot[eV]", "Epot[eV]", "Ekin[eV]", "T[K]")
    assert lines[1] == "%-10.4f %12.4f %12.4f %12.4f  %6.1f" % (0.0, -1.25, -1.5, 0.25, 300.0)
    assert len(lines) == 4
    bad = AsyncGPUMDLogger(tmpl, torch.device("cpu"), trajectory=_Failing(), state_dtype=torch.float64)
    bad.enqueue(step=0, time_ps=0.0, positions=z, momenta=z, forces=z.float(), cell=torch.eye(3),
                potential_energy=torch.tensor(0.0), kinetic_energy=torch.tensor(0.0), temperature=torch.tensor(0.0))
    with pytest.raises(RuntimeError, match="disk full"):
        bad.flush()
    bad.close()  # already reported: no second raise
    with pytest.raises(ValueError, match="EXTXYZ"):
        AsyncGPUMDLogger(tmpl, torch.device("cpu"), trajectory="frames.traj")


# ---------------------------------------------------------------------------------------- GPU
def _md(device, **kw):
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics
    from fastmd_amd.models.pair_potential import MorsePairAdapter

    return GPUResidentMolecularDynamics(systems.perovskite(3), model=MorsePairAdapter(device=device), device=device,
                                        temperature=500.0, timestep=0.25, tdamp=25.0,
                                        config=InferenceConfig(execution="whole_step"), steps_per_launch=10, **kw)


@pytest.mark.gpu
def test_whole_step_outputs_and_bitwise_resume(device, tmp_path):
    out = tmp_path / "run"
    ref = _md(device)
    ref.run(40)
    torch.cuda.synchronize()
    final = ref.integrator.state.flat.detach().cpu().clone()
    md = _md(device, output_dir=out, thermo_interval=10, xyz_interval=10, restart_interval=20, total_steps=40,
             trajectory=tmp_path / "log.xyz", logfile=tmp_path / "log.txt", loginterval=10)
    md.run(20)
    md.close()
    frames = mp.read_extxyz(out / mp.TRAJECTORY_FILE)
    assert [f["info"]["step"] for f in frames] == [0, 10, 20]
    assert frames[0]["keys"] == ["Lattice", "Properties", "step", "time_fs", "target_temp_K", "nhc_eta", "nhc_p_eta",
                                 "nhc_conserved_energy", "energy", "pbc"]
    # the frames of steps 10 and 20 are the CPU oracle's integrated states (tests/md_oracle.py)
    import md_oracle
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    s = systems.perovskite(3)
    o = md_oracle.run_nhc(s, md_oracle.morse_forces(s), maxwell_boltzmann_momenta(s.masses, 500.0, 0), 20,
                          sample_every=10, positions_until=20)
    for k in (1, 2):
        assert np.abs(frames[k]["positions"] - o["positions"][k]).max() < 1e-4
        assert np.abs(frames[k]["velocities"] - o["momenta"][k] / s.masses[:, None]).max() < 1e-6
        assert np.abs(frames[k]["forces"] - o["forces"][k]).max() < 1e-4
        assert np.array_equal(frames[k]["masses"], s.masses)
        assert abs(frames[k]["energy"] - o["energy"][k]) < 1e-6 * s.n_atoms
        assert abs(frames[k]["info"]["nhc_conserved_energy"] - o["conserved"][k]) < 1e-6 * s.n_atoms
    state = md.integrator
    assert np.allclose(frames[-1]["positions"], state.positions.cpu().numpy(), atol=1e-7)
    assert np.allclose(frames[-1]["forces"], state.forces.cpu().numpy(), atol=1e-7)
    thermo = (out / mp.THERMO_FILE).read_text().splitlines()
    assert thermo[0] + "\n" == mp.THERMO_HEADER and [int(t.split("\t")[0]) for t in thermo[1:]] == [10, 20]
    assert len((tmp_path / "log.txt").read_text().splitlines()) == 1 + 3  # header + steps 0, 10, 20
    assert len(mp.read_extxyz(tmp_path / "log.xyz")) == 3
    restart = mp.read_restart(out / mp.RESTART_FILE)
    assert restart.step == 20 and restart.offsets[mp.TRAJECTORY_FILE] == (out / mp.TRAJECTORY_FILE).stat().st_size
    # the continuation: same trajectory as the uninterrupted run, bitwise; outputs appended
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics
    from fastmd_amd.models.pair_potential import MorsePairAdapter

    cont = GPUResidentMolecularDynamics.from_restart(
        out / mp.RESTART_FILE, MorsePairAdapter(device=device), device=device, temperature=500.0, timestep=0.25,
        tdamp=25.0, config=InferenceConfig(execution="whole_step"), steps_per_launch=10, output_dir=out,
        thermo_interval=10, xyz_interval=10, restart_interval=20, total_steps=40)
    assert cont.nsteps == 20
    cont.run(20)
    cont.close()
    torch.cuda.synchronize()
    assert torch.equal(cont.integrator.state.flat.detach().cpu(), final)
    assert [f["info"]["step"] for f in mp.read_extxyz(out / mp.TRAJECTORY_FILE)] == [0, 10, 20, 30, 40]
    assert [int(t.split("\t")[0]) for t in (out / mp.THERMO_FILE).read_text().splitlines()[1:]] == [10, 20, 30, 40]
    th = cont.thermodynamics()
    assert th["step"] == 40 and abs(th["total_energy"] - th["potential_energy"] - th["kinetic_energy"]) < 1e-9
