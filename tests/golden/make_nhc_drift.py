"""Writes the CPU-oracle NHC trajectories the GPU drift gates compare against (test infrastructure).

    python tests/golden/make_nhc_drift.py            # the three fixtures (about 20 minutes on 8 cores)
    python tests/golden/make_nhc_drift.py morse      # only nhc_drift_morse_135.npz
    python tests/golden/make_nhc_drift.py mace_like_10k   # only nhc_drift_mace_like_135_10k.npz

Both runs integrate the 135-atom perovskite (3 x 3 x 3 cells, jitter 0.05 A, seed 0) under
NVT-NHC at 500 K (dt 0.25 fs, tdamp 25 fs, tchain 3, tloop 1, float32 kick) with the
Maxwell-Boltzmann momenta of seeds 0, 1 and 2, with forces from ``tests/md_oracle.py``:

* ``nhc_drift_morse_135.npz``: the configs[0] Morse potential, 10 000 steps, C(t) every 100 steps.
* ``nhc_drift_mace_like_135.npz``: configs[2], the random-init (seed 0) 2-layer 128-channel
  MACE-like model, 2 000 steps, C(t) every 10 steps, once with the model in float64 and once in
  float32 (the arithmetic class of the reference's model path); positions at steps 0, 10, .., 50
  of the float64 runs.
* ``nhc_drift_mace_like_135_10k.npz``: the same model and runs over 10 000 steps, C(t) every 50
  steps, float32 and float64 (the six runs in parallel processes, one thread each).

The tests pin each fixture to a short live run of the oracle (``tests/test_nhc_drift.py``).
"""
from __future__ import annotations

import dataclasses
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for path in (ROOT, os.path.dirname(HERE)):
    if path not in sys.path:
        sys.path.insert(0, path)

SEEDS = (0, 1, 2)
MORSE_STEPS, MORSE_EVERY = 10_000, 100
MACE_STEPS, MACE_EVERY, MACE_POSITIONS_UNTIL = 2_000, 10, 50
MACE_LONG_STEPS, MACE_LONG_EVERY = 10_000, 50


def mace_params():
    from fastmd_amd.models.mace_like import MaceLike, MaceLikeConfig

    cfg = MaceLikeConfig()
    model = MaceLike(cfg)
    return {k: v.detach().clone() for k, v in model.named_parameters()}, dataclasses.asdict(cfg)


def morse_runs():
    import md_oracle
    from fastmd_amd import systems
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    s = systems.perovskite(3)
    series = []
    for seed in SEEDS:
        out = md_oracle.run_nhc(s, md_oracle.morse_forces(s), maxwell_boltzmann_momenta(s.masses, 500.0, seed),
                                MORSE_STEPS, sample_every=MORSE_EVERY)
        series.append(out["conserved"])
        print(f"morse seed {seed}: max drift {md_oracle.max_drift(out['conserved']):.3e} eV", flush=True)
    np.savez_compressed(os.path.join(HERE, "nhc_drift_morse_135.npz"), seeds=np.array(SEEDS), steps=out["steps"],
                        conserved=np.stack(series))


def mace_runs():
    import torch

    import md_oracle
    from fastmd_amd import systems
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    params, cfg = mace_params()
    s = systems.perovskite(3)
    result = {}
    for name, dtype in (("f64", torch.float64), ("f32", torch.float32)):
        series, positions = [], []
        for seed in SEEDS:
            t0 = time.time()
            out = md_oracle.run_nhc(s, md_oracle.mace_like_forces(s, params, cfg, dtype=dtype),
                                    maxwell_boltzmann_momenta(s.masses, 500.0, seed), MACE_STEPS,
                                    sample_every=MACE_EVERY, positions_until=MACE_POSITIONS_UNTIL)
            series.append(out["conserved"])
            positions.append(out["positions"])
            print(f"mace_like {name} seed {seed}: max drift {md_oracle.max_drift(out['conserved']):.3e} eV "
                  f"({time.time() - t0:.0f} s)", flush=True)
        result[f"conserved_{name}"] = np.stack(series)
        if name == "f64":
            result["positions_f64"] = np.stack(positions)
    np.savez_compressed(os.path.join(HERE, "nhc_drift_mace_like_135.npz"), seeds=np.array(SEEDS),
                        steps=out["steps"], **result)


def _mace_long_run(task):
    """One 10 000-step MACE-like run (dtype name, seed) in a worker process: C(t) every 50 steps."""
    import torch

    torch.set_num_threads(1)
    import md_oracle
    from fastmd_amd import systems
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta

    name, seed = task
    params, cfg = mace_params()
    s = systems.perovskite(3)
    dtype = torch.float64 if name == "f64" else torch.float32
    t0 = time.time()
    out = md_oracle.run_nhc(s, md_oracle.mace_like_forces(s, params, cfg, dtype=dtype),
                            maxwell_boltzmann_momenta(s.masses, 500.0, seed), MACE_LONG_STEPS,
                            sample_every=MACE_LONG_EVERY)
    print(f"mace_like 10k {name} seed {seed}: max drift {md_oracle.max_drift(out['conserved']):.3e} eV "
          f"({time.time() - t0:.0f} s)", flush=True)
    return name, seed, out["steps"], out["conserved"]


def mace_long_runs():
    import multiprocessing

    tasks = [(name, seed) for name in ("f32", "f64") for seed in SEEDS]
    with multiprocessing.get_context("spawn").Pool(len(tasks)) as pool:
        results = pool.map(_mace_long_run, tasks)
    by = {(name, seed): conserved for name, seed, _, conserved in results}
    steps = results[0][2]
    np.savez_compressed(os.path.join(HERE, "nhc_drift_mace_like_135_10k.npz"), seeds=np.array(SEEDS), steps=steps,
                        conserved_f32=np.stack([by["f32", seed] for seed in SEEDS]),
                        conserved_f64=np.stack([by["f64", seed] for seed in SEEDS]))


if __name__ == "__main__":
    which = sys.argv[1:] or ["morse", "mace_like", "mace_like_10k"]
    if "morse" in which:
        morse_runs()
    if "mace_like" in which:
        mace_runs()
    if "mace_like_10k" in which:
        mace_long_runs()
