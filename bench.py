"""Benchmark of the MI355X-native GPU-resident MD step (one JSON line on stdout).

Metric: "MD ms/step & atom-steps/s (whole_step) at 135/10k atoms; segment_sum
HBM GB/s". The headline ``value`` is whole-step MD throughput in atom-steps/s on the 10 000-atom
perovskite (10 x 10 x 20 cells, configs[3]) with the random-init 2-layer 128-channel MACE-like
model, NVT Nose-Hoover chain at 500 K (tdamp 25 fs, tchain 3, tloop 1, dt 0.25 fs); the
135-atom system and the segment-sum microbenchmark (configs[1], 40 000 atoms,
F = 128) are reported beside it, with the dominant kernel's roofline and the CPU baseline (the
PyTorch-CPU eager oracle on this host's cores, a bounded sample of the same workload).

  python bench.py [--gpus 1] [--steps 200] [--warmup 3] [--no-cpu] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "MD ms/step & atom-steps/s (whole_step) at 135/10k atoms; segment_sum HBM GB/s"
HBM_PEAK_GBPS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
STEPS_PER_LAUNCH = 10


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_md(n_atoms: int, steps_per_launch: int):
    import torch

    from fastmd_amd import systems
    from fastmd_amd.config import InferenceConfig
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics
    from fastmd_amd.models.mace_like import MaceLikeAdapter

    device = torch.device("cuda", 0)
    s = systems.perovskite_atoms(n_atoms)
    return GPUResidentMolecularDynamics(s, model=MaceLikeAdapter(device=device), device=device, temperature=500.0,
                                        timestep=0.25, tdamp=25.0, tchain=3, tloop=1,
                                        config=InferenceConfig(execution="whole_step"),
                                        steps_per_launch=steps_per_launch)


def time_md(md, steps: int, warmup_windows: int) -> float:
    """Seconds for exactly ``steps`` MD steps (barrier + synchronize on both sides)."""
    import torch

    md.run(warmup_windows * md.steps_per_launch)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    md.run(steps)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def time_kernel(fn, reps: int = 20) -> float:
    """Average duration (s) of ``fn``'s launches between HIP events on torch's current stream
    (the stream the kernels are launched on)."""
    import torch

    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / reps


def gemm_roofline(md) -> dict:
    """The dominant kernel of the 10 000-atom step, the fp32 MFMA edge GEMM z = a @ W1
    ([e_cap, 2C+8] x [2C+8, 4C]), timed live; algorithmic flops = 2 M K N per launch."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm

    layer = md.adapter.module.layers[0]
    m = md.whole_step_runner.builder.e_capacity
    k, n = layer.W1.shape
    a = torch.randn(m, k, device=md.device)
    out = torch.empty(m, n, device=md.device)
    t = time_kernel(lambda: gemm(a, layer.W1, b_layout=1, out=out))
    flops = 2.0 * m * k * n
    achieved = flops / t / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": None, "kernel": "gemm_f32_kernel<1>",
            "launch_ms": round(t * 1e3, 4), "flops_per_launch": flops, "shape": [m, k, n]}


def segment_sum_bench(n_atoms: int = 40000, F: int = 128) -> dict:
    """configs[1] segment sum [E, F] -> [N, F] over the sorted (identity) CSR of the 40 000-atom
    perovskite at rc = 6 A; algorithmic bytes E F 4 + N F 4 + (N + 1) 8."""
    import torch

    from fastmd_amd import systems
    from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder
    from fastmd_amd.ops.csr_segment_sum import Csr, segment_sum_csr

    device = torch.device("cuda", 0)
    s = systems.perovskite_atoms(n_atoms)
    g = TensorGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers), atom_graph_cutoff=6.0,
                           device=device, check_isolated_atoms=False).build(torch.tensor(s.positions, device=device))
    e = int(g.n_edges.item())
    gen = torch.Generator(device="cpu").manual_seed(0)
    v = torch.randn(e, F, generator=gen).to(device)
    out = torch.empty(n_atoms, F, device=device)
    csr = Csr(g.edge_offsets)
    t = time_kernel(lambda: segment_sum_csr([(v, csr, 0, 1.0, None)], n_atoms, F, out=out), reps=50)
    nbytes = e * F * 4 + n_atoms * F * 4 + (n_atoms + 1) * 8
    gbps = nbytes / t / 1e9
    return {"segment_sum_GBps": round(gbps, 1), "segment_sum_frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4),
            "segment_sum_us": round(t * 1e6, 2), "segment_sum_edges": e, "segment_sum_F": F,
            "segment_sum_atoms": n_atoms}


def cpu_baseline(n_atoms: int, budget_s: float) -> dict:
    """The CPU oracle (PyTorch-CPU eager model forward+backward with index_select/index_add_/matmul,
    NumPy neighbour list and NHC) on this host, whole MD steps until ``budget_s`` elapsed."""
    import numpy as np
    import torch

    from oracle import models as om
    from oracle import nhc as onhc
    from oracle import nl as onl
    from fastmd_amd import systems
    from fastmd_amd.execution.gpu_nhc import maxwell_boltzmann_momenta
    from fastmd_amd.models.mace_like import MaceLike, MaceLikeConfig

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    s = systems.perovskite_atoms(n_atoms)
    cfg = MaceLikeConfig()
    model = MaceLike(cfg)
    params = {k: v.detach().clone() for k, v in model.named_parameters()}
    cdict = {f: getattr(cfg, f) for f in cfg.__dataclass_fields__}
    elem_of = {z: k for k, z in enumerate(cfg.elements)}
    elem = torch.tensor([elem_of[int(z)] for z in s.numbers])
    cell32 = s.cell.astype(np.float32)
    inv = np.linalg.inv(cell32.astype(np.float64)).astype(np.float32)
    cell_t = torch.tensor(cell32)

    def forces(q):
        _, wraps, wrapped = onl.wrap(q, inv, cell32)
        cand = onl.candidates(wrapped, cell32, np.float32(36.0 + 1e-3), 200)
        b = onl.build(q, inv, cell32, cand, q.astype(np.float32), wraps, np.float32(36.0), np.float32(1.0),
                      (1, 0, 0), int(cand.num_neighbors.sum()))
        e = b.n_edges
        fn = lambda pos: om.mace_like_node_energy(params, cdict, pos, cell_t, elem,
                                                  torch.tensor(b.center[:e].astype(np.int64)),
                                                  torch.tensor(b.neighbor[:e].astype(np.int64)),
                                                  torch.tensor(b.images[:e]))
        energy, f, _ = om.energy_and_forces(fn, torch.tensor(b.wrapped))
        return f.numpy(), float(energy)

    p0 = maxwell_boltzmann_momenta(s.masses, 500.0, seed=0)
    f0, e0 = forces(s.positions)
    o = onhc.NHC(s.masses, s.positions, p0, temperature_K=500.0, timestep=0.25 * onhc.FS, tdamp=25 * onhc.FS,
                 f32_kick=True, forces=f0, energy=e0)
    steps = 0
    t0 = time.perf_counter()
    while True:
        o.step(forces)
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s:
            break
    return {"value": round(n_atoms * steps / elapsed, 1), "unit": "atom-steps/s", "cores": threads,
            "kind": "port", "ms_per_step": round(elapsed / steps * 1e3, 2),
            "sample": f"{steps} whole MD steps (neighbour list + MACE-like forward/backward + NHC) of the "
                      f"{n_atoms}-atom perovskite in PyTorch-CPU eager / NumPy, fp32 model, fp64 integrator"}


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--steps-small", type=int, default=2000)
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--cpu-seconds", type=float, default=15.0)
    parser.add_argument("--quick", action="store_true", help="short run (profiling): no CPU baseline, fewer steps")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs the MD step on one MI355X; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is a design only, see DESIGN.md)", file=sys.stderr)
        return 2
    if args.steps % STEPS_PER_LAUNCH:
        print(f"--steps must be a multiple of {STEPS_PER_LAUNCH}", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    steps_small = 200 if args.quick else args.steps_small

    log("10 000 atoms: capture")
    md = build_md(10000, STEPS_PER_LAUNCH)
    log("10 000 atoms: timing")
    t_big = time_md(md, args.steps, args.warmup)
    ms_big = t_big / args.steps * 1e3
    stats_big = md.whole_step_stats()
    log(f"10 000 atoms: {ms_big:.3f} ms/step")
    roof = gemm_roofline(md)
    del md
    torch.cuda.empty_cache()

    log("135 atoms: capture")
    md = build_md(135, STEPS_PER_LAUNCH)
    t_small = time_md(md, steps_small, args.warmup)
    ms_small = t_small / steps_small * 1e3
    stats_small = md.whole_step_stats()
    log(f"135 atoms: {ms_small:.4f} ms/step")
    del md
    torch.cuda.empty_cache()

    log("segment sum microbenchmark")
    seg = segment_sum_bench()
    cpu = None
    if not (args.no_cpu or args.quick):
        log("CPU baseline (oracle)")
        cpu = cpu_baseline(10000, args.cpu_seconds)
        cpu135 = cpu_baseline(135, min(5.0, args.cpu_seconds))
        cpu["ms_per_step_135"] = cpu135["ms_per_step"]
    line = {
        "metric": METRIC,
        "value": round(10000 / (ms_big / 1e3), 1),
        "unit": "atom-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_big, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded jittered CsSnI3-like perovskite, random-init (seed 0) MACE-like model",
        "config": {"workload": "whole_step NVT-NHC MD (500 K, dt 0.25 fs, tdamp 25 fs, tchain 3, tloop 1), "
                               "2-layer 128-channel L1 correlation-3 MACE-like model, 8 Bessel, rc 6 A, "
                               "10 000-atom perovskite (10x10x20 cells)",
                   "atoms": 10000, "steps_per_launch": STEPS_PER_LAUNCH,
                   "e_capacity": stats_big["e_capacity"]},
        "roofline": roof,
        "cpu_baseline": cpu,
        "md_steps_per_s": round(1e3 / ms_big, 2),
        "small_system": {"atoms": 135, "ms_per_step": round(ms_small, 5), "md_steps_per_s": round(1e3 / ms_small, 1),
                         "atom_steps_per_s": round(135 / (ms_small / 1e3), 1), "steps": steps_small,
                         "e_capacity": stats_small["e_capacity"]},
        "segment_sum": seg,
        "whole_step_stats_10k": {k: stats_big[k] for k in ("candidate_refreshes", "fallback_windows",
                                                           "max_edge_count", "capacity_history")},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
