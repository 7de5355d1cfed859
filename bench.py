"""Benchmark of the MI355X-native GPU-resident MD step (one JSON line on stdout).

Metric: "MD ms/step & atom-steps/s (whole_step) at 135/10k atoms; segment_sum
HBM GB/s". The headline ``value`` is whole-step MD throughput in atom-steps/s on the 10 000-atom
perovskite (10 x 10 x 20 cells, configs[3]) with the random-init 2-layer 128-channel MACE-like
model, NVT Nose-Hoover chain at 500 K (tdamp 25 fs, tchain 3, tloop 1, dt 0.25 fs); the
135-atom system and the segment-sum microbenchmark (configs[1], 40 000 atoms,
F = 128) are reported beside it, with the dominant kernel's roofline and the CPU baseline (the
PyTorch-CPU eager oracle on this host's cores, a bounded sample of the same workload).

  python bench.py [--gpus 1] [--steps 1000] [--warmup 1000] [--no-cpu] [--quick] [--ops] [--scaling] [--nhc]
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
# VALU issue peak: 256 CUs x 4 SIMDs x 2.4 GHz, one wave64 VALU instruction per 4 cycles per SIMD
# (16 lanes wide; full-rate 32-bit operations)
VALU_ISSUE_PEAK_GINSTS = 256 * 4 * 2.4 / 4
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
SPLIT_PRODUCTS = 6  # fp32-accurate GEMM: three bf16 planes per operand, six MFMA products
SPIN_CYCLES = 20_000_000  # GPU clock cycles of torch.cuda._sleep (several ms)
ROOFLINE_KERNEL = "message_bwd_edge_kernel<2, true, 8, true, 1>"
STEPS_PER_LAUNCH = 10


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_md(n_atoms: int, steps_per_launch: int, bond_cutoff: float | None = None, execution: str = "whole_step",
             **outputs):
    """The MD of a perovskite (whole-step by default): the MACE-like model, or with
    ``bond_cutoff`` the configs[4] three-body model (64 channels, 4 layers, that bond cutoff)."""
    import torch

    from fastmd_amd import systems
    from fastmd_amd.config import InferenceConfig
    from fastmd_amd.interfaces.gpu_md import GPUResidentMolecularDynamics
    from fastmd_amd.models.mace_like import MaceLikeAdapter
    from fastmd_amd.models.threebody_like import ThreeBodyAdapter, ThreeBodyConfig

    device = torch.device("cuda", 0)
    s = systems.perovskite_atoms(n_atoms)
    model = (MaceLikeAdapter(device=device) if bond_cutoff is None else
             ThreeBodyAdapter(config=ThreeBodyConfig(bond_cutoff=bond_cutoff), device=device))
    return GPUResidentMolecularDynamics(s, model=model, device=device, temperature=500.0,
                                        timestep=0.25, tdamp=25.0, tchain=3, tloop=1,
                                        config=InferenceConfig(execution=execution),
                                        steps_per_launch=steps_per_launch, **outputs)


def time_md(md, steps: int, warmup_steps: int, thermalise: int = 0) -> float:
    """Seconds for exactly ``steps`` MD steps after ``thermalise`` untimed equilibration steps (the
    random-init potential keeps adding edges for about 2 000 steps from the jittered lattice, each
    growth a recapture) and then ``warmup_steps`` untimed ones (each rounded up to whole windows),
    synchronized on both sides (one process, one GPU: no barrier to take)."""
    import torch

    spl = md.steps_per_launch
    if thermalise > 0:
        md.run(-(-thermalise // spl) * spl)
    md.run(-(-warmup_steps // spl) * spl)
    before = md.whole_step_stats()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    md.run(steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    after = md.whole_step_stats()
    # events inside the timed region (each is part of the measured time)
    md.timed_events = {"capacity_growths": len(after["capacity_history"]) - len(before["capacity_history"]),
                       "fallback_windows": after["fallback_windows"] - before["fallback_windows"],
                       "candidate_refreshes": after["candidate_refreshes"] - before["candidate_refreshes"]}
    return elapsed


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


def message_roofline(md) -> dict:
    """The dominant kernel of the 10 000-atom step: the second layer's edge-side message VJP
    (message_bwd_edge_kernel, node-factored pre-activation: per row the sender's P, h0, h1 rows
    gathered, z rebuilt with the radial term, its gradient, the radial-basis and geometry
    gradients; per atom the centre's Q, gA0, gA1 read and the sum of g_z written). It is timed
    in the context of the step: HIP events on torch's current stream (the stream it is launched
    on) around that launch alone in eager force evaluations at the run's final state (its edge
    list and features), the launch split out of the model's combined VJP call here. Ten times, a spin kernel is queued and then
    two evaluations behind it, so that no host latency falls inside the event pairs; the second
    evaluation of each pair is timed (its launch follows the same kernels as in the captured
    step, with their data in L2), the first is reported as ``first_launch_us``.
    Algorithmic bytes per launch, counted as the gather-cat's formula counts them (every
    gathered row once per edge that reads it): per real edge row 4 B neighbour index + 20 B
    geometry (unit vector, length, cutoff) + 4 nb B basis + 4 (NZ + 4) C B of gathered sender
    rows (P: NZ C, h0: C, h1: 3 C) + 16 B geometry-gradient store + 4 nb B basis-gradient store;
    per atom 20 B offsets and order + 4 (NZ + 4) C B read (Q, gA0, gA1) + 4 NZ C B stored
    (the per-centre sum of g_z), NZ = 4 (the last layer has vector features). The
    ``unique_bytes`` alternative counts every input row once (a perfect cache).
    The kernel is bound by instruction issue, not by HBM: ``bound`` "valu", ``achieved`` its VALU
    wave-instructions per second (the committed SQ_INSTS_VALU count per launch over the live
    launch time) against the issue peak of one wave64 VALU instruction per 4 cycles per SIMD;
    ``hbm_frac`` is its measured HBM traffic (FETCH_SIZE + WRITE_SIZE) over the launch time and
    ``gather_bytes_frac`` the gather-cat byte count's rate, both as fractions of 8 TB/s."""
    import torch

    from fastmd_amd.models import mace_like

    runner = md.whole_step_runner
    torch.cuda.synchronize()
    time.sleep(0.03)  # an idle gap that separates the timed steps from these launches in a kernel trace
    events = []
    launch = mace_like._call

    def timed_call(name, *args):
        # The model's VJP launches both message VJP kernels in one fmd_mace_message_bwd_f32 call
        # (arguments as in include/fastmd_hip.h: 18 gzsum_src, 21 gh0, 22 gh1, 23 accumulate_h).
        # The call that carries gzsum_src (the last layer's) is split here into the edge-side
        # kernel alone between HIP events (no gzsum_src, gh0, gh1) and then the sender-side kernel
        # alone (accumulate_h bit 2): the same kernels and results as the single call.
        if name != "fmd_mace_message_bwd_f32" or args[18] is None or torch.cuda.is_current_stream_capturing():
            return launch(name, *args)
        edge = list(args)
        edge[18] = edge[21] = edge[22] = None
        edge[23] = 0
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        ev[0].record()
        launch(name, *edge)
        ev[1].record()
        events.append((ev[0], ev[1], (args[7], args[8], args[10])))
        src = list(args)
        src[23] = args[23] | 4
        return launch(name, *src)

    mace_like._call = timed_call
    try:
        for _ in range(10):
            # a spin kernel ahead of each pair of evaluations keeps the GPU busy while the host
            # enqueues their launches, so the GPU runs them back to back as in the captured step
            torch.cuda._sleep(SPIN_CYCLES)
            runner._evaluate(md.integrator.positions)
            runner._evaluate(md.integrator.positions)
        torch.cuda.synchronize()
    finally:
        mace_like._call = launch
    e_cap, n, C = events[-1][2]
    if len(events) != 20 or any(shape != (e_cap, n, C) for _, _, shape in events):
        raise RuntimeError("the roofline evaluations ran on different edge capacities")
    durations = [a.elapsed_time(b) / 1e3 for a, b, _ in events]
    first = durations[0::2]
    durations = durations[1::2]
    t = sum(durations) / len(durations)
    edges = int(runner.builder.edge_offsets[-1].item())
    rows = min(edges, e_cap)
    nb, nz = md.adapter.module.config.n_basis, 4
    per_row = 4 + 20 + 4 * nb + 4 * (nz + 4) * C + 16 + 4 * nb
    per_atom = 20 + 4 * (nz + 4) * C + 4 * nz * C
    gathered = rows * per_row + n * per_atom
    unique = rows * (4 + 20 + 4 * nb + 16 + 4 * nb) + n * (20 + 4 * (nz + 4) * C + 4 * nz * C + 4 * (nz + 4) * C)
    counters = _counters(ROOFLINE_KERNEL, [rows, n, C])
    traffic = counters.get("bytes_per_launch")
    insts = counters.get("valu_insts_per_launch")
    out = {"kernel": ROOFLINE_KERNEL, "launch_us": round(t * 1e6, 2), "launches_timed": len(durations),
           "first_launch_us": round(sum(first) / len(first) * 1e6, 2), "rows": rows, "atoms": n,
           "traffic": traffic,
           "hbm_frac": None if traffic is None else round(traffic / t / 1e9 / HBM_PEAK_GBPS, 4),
           "gather_bytes_per_launch": gathered,
           "gather_bytes_frac": round(gathered / t / 1e9 / HBM_PEAK_GBPS, 4),
           "gather_bytes_basis": f"per real edge row {per_row} B (gathered sender rows counted per row), per atom "
                                 f"{per_atom} B",
           "unique_bytes_per_launch": unique, "unique_frac": round(unique / t / 1e9 / HBM_PEAK_GBPS, 4)}
    if insts is not None:
        # the kernel is bound by instruction issue (its HBM traffic is a small fraction of the peak)
        achieved = insts / t / 1e9
        out.update(bound="valu", achieved=round(achieved, 1), peak=VALU_ISSUE_PEAK_GINSTS, unit="Ginst/s",
                   frac=round(achieved / VALU_ISSUE_PEAK_GINSTS, 4), valu_insts_per_launch=insts,
                   mfma_insts_per_launch=counters.get("mfma_insts_per_launch"))
    else:
        achieved = unique / t / 1e9
        out.update(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBPS, unit="GB/s",
                   frac=round(achieved / HBM_PEAK_GBPS, 4))
    return out


def _counters(kernel: str, shape: list) -> dict:
    """Per-launch counter figures of ``kernel`` at ``shape`` from the committed rocprofv3 --pmc
    summary (profiles/traffic.json): HBM bytes (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel
    calibration) and, where measured, VALU and MFMA instructions (SQ_INSTS_VALU, SQ_INSTS_MFMA),
    each scaled from the measured shape to this launch's rows; {} if no entry matches."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return {}
    row = table.get(kernel)
    if not row or row.get("shape", [None])[1:] != shape[1:]:
        return {}
    scale = shape[0] / row["shape"][0]  # the per-row work scales with the rows of the launch
    return {key: int(row[src] * scale) for key, src in (("bytes_per_launch", "bytes_per_launch"),
                                                        ("valu_insts_per_launch", "valu_insts"),
                                                        ("mfma_insts_per_launch", "mfma_insts")) if src in row}


def hbm_ops_bench(n_atoms: int = 40000, F: int = 128, gemm: bool = False) -> dict:
    """configs[1] memory-bound operators on the perovskite of ``n_atoms`` atoms at rc = 6 A (sorted
    edge list, 15.2 edges/atom), width F, fp32, each timed live with HIP events. Two byte counts
    per op: ``hbm_bytes``, every input row read once and every output written once (the HBM
    traffic a perfect cache gives; ``GBps`` and ``frac_of_hbm_peak`` use it), and
    ``survey_bytes``, the per-gathered-load formula, which counts a source row once per edge
    that reads it (those re-reads are L2/MALL hits, so its rate can exceed the HBM peak):
      segment_sum [E,F] -> [N,F]:      hbm = survey = E F 4 + N F 4 + (N + 1) 8
      transpose   [N,F] -> [E,F]:      hbm = E F 4 + N F 4 + (N + 1) 8;  survey = 2 E F 4 + E 4
      gather_cat  [E, 2F + 8]:         hbm = E (2F + 8) 4 + N F 4 + E 8 4 + E 2 4;  survey = E (16 F + 72)
    With ``gemm`` the wide edge GEMM [E, 2F + 8] x [2F + 8, 4F] is timed too (fp32-accurate on
    prebuilt rows, the same with the gather-cat fused into its operand load, and bf16 operands;
    fp32 out; flops 2 E (2F + 8) 4F)."""
    import torch

    from fastmd_amd import systems
    from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder
    from fastmd_amd.models.mace_like import _gather_edge_rows
    from fastmd_amd.ops.csr_segment_sum import Csr, segment_sum_csr, segment_sum_t
    from fastmd_amd.ops.wide_gemm import gemm as wide_gemm
    from fastmd_amd.ops.wide_gemm import gemm_gather

    device = torch.device("cuda", 0)
    s = systems.perovskite_atoms(n_atoms)
    g = TensorGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers), atom_graph_cutoff=6.0,
                           line_graph_cutoff=None, device=device, check_isolated_atoms=False).build(torch.tensor(s.positions, device=device))
    e = int(g.n_edges.item())
    gen = torch.Generator(device="cpu").manual_seed(0)
    v = torch.randn(e, F, generator=gen).to(device)
    x = torch.randn(n_atoms, F, generator=gen).to(device)
    rbf = torch.randn(e, 8, generator=gen).to(device)
    out = torch.empty(n_atoms, F, device=device)
    rows = torch.empty(e, 2 * F + 8, device=device)
    csr = Csr(g.edge_offsets)
    ei = g.edge_index[:e]
    res = {"atoms": n_atoms, "edges": e, "F": F}
    reps = 50 if e > 100000 else 200

    def put(name, t, hbm, survey):
        gbps = hbm / t / 1e9
        res[name] = {"us": round(t * 1e6, 2), "GBps": round(gbps, 1), "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4),
                     "hbm_bytes": hbm, "survey_bytes": survey, "survey_GBps": round(survey / t / 1e9, 1)}

    seg_bytes = e * F * 4 + n_atoms * F * 4 + (n_atoms + 1) * 8
    put("segment_sum", time_kernel(lambda: segment_sum_csr([(v, csr, 0, 1.0, None)], n_atoms, F, out=out), reps=reps),
        seg_bytes, seg_bytes)
    put("segment_sum_transpose", time_kernel(lambda: segment_sum_t(x, csr, e), reps=reps), seg_bytes,
        2 * e * F * 4 + e * 4)
    put("gather_cat", time_kernel(lambda: _gather_edge_rows(x, rbf, ei, rows), reps=reps),
        e * (2 * F + 8) * 4 + n_atoms * F * 4 + e * 8 * 4 + e * 2 * 4, e * (16 * F + 72))
    if gemm:
        k, n = 2 * F + 8, 4 * F
        w = torch.randn(k, n, generator=gen).to(device) / k ** 0.5
        flops = 2.0 * e * k * n
        z = torch.empty(e, n, device=device)
        wt = w.t().contiguous()  # [4F, 2F+8]: the weight layout of F.linear (K-contiguous)
        t32 = time_kernel(lambda: wide_gemm(rows, wt, b_layout=0, out=z), reps=reps)
        tfused = time_kernel(lambda: gemm_gather([(x, ei[:, 1]), (x, ei[:, 0]), (rbf, None)], wt, out=z), reps=reps)
        rows16, w16 = rows.to(torch.bfloat16), wt.to(torch.bfloat16)
        t16 = time_kernel(lambda: wide_gemm(rows16, w16, b_layout=0, out=z), reps=reps)
        split_peak = BF16_MFMA_PEAK_TFLOPS / SPLIT_PRODUCTS
        for name, t in (("edge_gemm_f32", t32), ("gather_cat_edge_gemm_f32_fused", tfused)):
            res[name] = {"us": round(t * 1e6, 2), "TFLOPs": round(flops / t / 1e12, 2),
                         "frac_of_split_ceiling": round(flops / t / 1e12 / split_peak, 4),
                         "frac_of_fp32_mfma_peak": round(flops / t / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4)}
        b16 = 2 * (e * k + k * n) + 4 * e * n
        res["edge_gemm_bf16"] = {"us": round(t16 * 1e6, 2), "TFLOPs": round(flops / t16 / 1e12, 2),
                                 "GBps": round(b16 / t16 / 1e9, 1),
                                 "frac_of_hbm_peak": round(b16 / t16 / 1e9 / HBM_PEAK_GBPS, 4)}
    return res


def ops_sweep() -> list:
    """every (N, F) of the operator microbenchmark."""
    out = []
    for n_atoms in (135, 3430, 40000):
        for F in (64, 128, 256):
            r = hbm_ops_bench(n_atoms, F, gemm=True)
            log(f"ops N={n_atoms} F={F}: " + ", ".join(
                f"{k} {r[k]['us']} us" for k in r if isinstance(r[k], dict)))
            out.append(r)
    return out


def scaling_sweep(steps: int, warmup: int) -> list:
    """the configs[2] model and 500 K NHC on k x k x k perovskite supercells,
    k in {3, 6, 10, 15, 20} (135 .. 40 000 atoms), ``steps`` whole-step steps each after ``warmup``
    untimed ones; beside each, the ragged (eager) builder at max_neighbors = 96 (one build) and
    forced through its overflow-rebuild path from 8 slots (the slot count grows, the edges are
    identical)."""
    import torch

    from fastmd_amd import systems
    from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder

    out = []
    for k in (3, 6, 10, 15, 20):
        n_atoms = 5 * k ** 3
        md = build_md(n_atoms, STEPS_PER_LAUNCH)
        t = time_md(md, steps, warmup)
        stats = md.whole_step_stats()
        row = {"k": k, "atoms": n_atoms, "steps": steps, "ms_per_step": round(t / steps * 1e3, 4),
               "md_steps_per_s": round(steps / t, 1), "atom_steps_per_s": round(n_atoms * steps / t, 1),
               "e_capacity": stats["e_capacity"], "timed_events": md.timed_events}
        del md
        torch.cuda.empty_cache()
        s = systems.perovskite(k)
        pos = torch.tensor(s.positions, device="cuda")
        for slots, key in ((96, "ragged_build_96"), (8, "ragged_build_overflow_from_8")):
            def build(slots=slots):
                b = TensorGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers),
                                       atom_graph_cutoff=6.0, line_graph_cutoff=None, device="cuda",
                                       max_neighbors=slots)
                g = b.build(pos)
                return b, g
            build()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            b, g = build()
            torch.cuda.synchronize()
            row[key] = {"ms": round((time.perf_counter() - t0) * 1e3, 3), "slots_after": b.max_neighbors,
                        "edges": int(g.n_edges.item())}
        log(f"scaling k={k} N={n_atoms}: {row['ms_per_step']} ms/step, ragged {row['ragged_build_96']}")
        out.append(row)
    return out


def threebody_bench(steps: int, warmup: int) -> list:
    """the three-body model on the 5 000-atom perovskite (10 x 10 x 10 cells), 500 K NHC,
    at the stated 3 A bond cutoff and at 3.5 A (where the B-X bonds, 3.1 A, enter the line graph)."""
    import torch

    out = []
    for rb in (3.0, 3.5):
        md = build_md(5000, STEPS_PER_LAUNCH, bond_cutoff=rb)
        t = time_md(md, steps, warmup)
        b = md.whole_step_runner.builder
        stats = md.whole_step_stats()
        row = {"atoms": 5000, "bond_cutoff": rb, "steps": steps, "warmup": warmup,
               "ms_per_step": round(t / steps * 1e3, 4), "md_steps_per_s": round(steps / t, 1),
               "atom_steps_per_s": round(5000 * steps / t, 1), "edges": int(b.edge_offsets[-1].item()),
               "bonds": int(b.short_offsets[-1].item()), "triplets": int(b.pair_offsets[-1].item()),
               "e_capacity": stats["e_capacity"], "t_capacity": b.t_capacity, "timed_events": md.timed_events}
        log(f"three-body rb={rb}: {row['ms_per_step']} ms/step, {row['bonds']} bonds, {row['triplets']} triplets")
        out.append(row)
        del md, b
        torch.cuda.empty_cache()
    return out


def frames_bench(steps: int, warmup: int) -> dict:
    """The reference's published protocol (S01, README.md:27-39): 135 atoms, whole-step NHC with an
    EXTXYZ trajectory frame every 10 steps (asynchronous device-to-host copies, writer thread),
    wall time per step including the output."""
    import tempfile

    import torch

    with tempfile.TemporaryDirectory() as tmp:
        md = build_md(135, STEPS_PER_LAUNCH, trajectory=os.path.join(tmp, "traj.xyz"), loginterval=10)
        md.run(-(-warmup // STEPS_PER_LAUNCH) * STEPS_PER_LAUNCH)
        md.logger.flush()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        md.run(steps)
        md.logger.flush()
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        md.close()
        size = os.path.getsize(os.path.join(tmp, "traj.xyz"))
    return {"atoms": 135, "steps": steps, "warmup": warmup, "frame_every": 10, "ms_per_step": round(t / steps * 1e3, 4),
            "md_steps_per_s": round(steps / t, 1), "trajectory_bytes": size}


def replica_bench(steps: int, warmup: int) -> list:
    """Replica batching (replica_batch.py): R replicas of the 135-atom configs[2] system (MACE-like,
    500 K NHC, their own momenta and chains) in one whole-step graph per window."""
    import torch

    from fastmd_amd import systems
    from fastmd_amd.execution.replica_batch import ReplicaBatchedMD
    from fastmd_amd.models.mace_like import MaceLikeAdapter

    out = []
    for replicas in (8, 32):
        md = ReplicaBatchedMD(systems.perovskite_atoms(135), MaceLikeAdapter(device="cuda"), replicas=replicas,
                              device="cuda", temperature=500.0, timestep=0.25, tdamp=25.0,
                              steps_per_launch=STEPS_PER_LAUNCH)
        md.run(-(-warmup // STEPS_PER_LAUNCH) * STEPS_PER_LAUNCH)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        md.run(steps)
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        row = {"replicas": replicas, "atoms_per_replica": 135, "steps": steps, "warmup": warmup,
               "ms_per_step": round(t / steps * 1e3, 4), "atom_steps_per_s": round(replicas * 135 * steps / t, 1),
               "capacity_history": md.capacity_history}
        log(f"replicas R={replicas}: {row['ms_per_step']} ms/step, {row['atom_steps_per_s']} atom-steps/s")
        out.append(row)
        del md
        torch.cuda.empty_cache()
    return out


def model_graph_bench(steps: int, warmup: int) -> list:
    """The model_graph execution mode (ragged build and integrator eager, the model's forward + VJP
    replayed per capacity bucket) of the MACE-like model at 135 and 10 000 atoms."""
    import torch

    out = []
    for n_atoms in (135, 10000):
        md = build_md(n_atoms, 1, execution="model_graph")
        md.run(warmup)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        md.run(steps)
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        st = md.model_graph_stats()
        row = {"atoms": n_atoms, "steps": steps, "warmup": warmup, "ms_per_step": round(t / steps * 1e3, 4),
               "atom_steps_per_s": round(n_atoms * steps / t, 1), "captures": st["captures"],
               "cached_buckets": st["cached_buckets"]}
        log(f"model_graph N={n_atoms}: {row['ms_per_step']} ms/step, {st['captures']} captures")
        out.append(row)
        del md
        torch.cuda.empty_cache()
    return out


def nhc_bench(sizes=(135, 10000, 40000), steps: int = 100, reps: int = 5) -> list:
    """The fused NHC velocity-Verlet halves alone (configs[0]/[2] 135 atoms, configs[3] 10 000 and
    40 000): ``steps`` steps (500 K, dt 0.25 fs, tdamp 25 fs, tchain 3, tloop 1, float32 forces)
    captured in one HIP graph and replayed ``reps`` times between HIP events, so the time is the
    kernels' alone. As the whole step runs them, a step's post-force half and the next step's
    pre-force half share a launch (``step_post_pre``: one workgroup up to 4 096 atoms, one launch;
    above, block partials with the chain run by the last workgroup, three launches); the separate
    pre-force + post-force pair is timed beside it (``us_per_step_separate``: two launches, or four
    above 4 096 atoms). Bytes per step as the survey counts them, 220 N (f64 positions, momenta,
    cached forces and masses read and written by the two halves, f32 forces read)."""
    import numpy as np
    import torch

    from fastmd_amd import systems, units
    from fastmd_amd.execution.gpu_nhc import GPUNoseHooverChainNVT, maxwell_boltzmann_momenta

    device = torch.device("cuda", 0)
    out = []
    for n in sizes:
        s = systems.perovskite_atoms(n)
        p0 = maxwell_boltzmann_momenta(s.masses, 500.0, seed=0)
        nhc = GPUNoseHooverChainNVT(s.masses, s.positions, np.asarray(p0, dtype=np.float64), temperature_K=500.0,
                                    timestep=0.25 * units.fs, tdamp=25.0 * units.fs, tchain=3, tloop=1,
                                    device=device, force_dtype=torch.float32)
        gen = torch.Generator(device="cpu").manual_seed(0)
        forces = (0.1 * torch.randn(n, 3, generator=gen)).to(device)
        energy = torch.zeros(1, dtype=torch.float64, device=device)

        def pair():
            nhc.step_pre_force()
            nhc.step_post_force(forces, energy=energy)

        def fused():
            nhc.step_post_pre(forces, energy=energy)

        def per_step_us(body) -> float:
            side = torch.cuda.Stream(device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                for _ in range(3):
                    body()
            torch.cuda.current_stream(device).wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(steps):
                    body()
            graph.replay()
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(reps):
                graph.replay()
            end.record()
            end.synchronize()
            del graph
            return start.elapsed_time(end) * 1e3 / (reps * steps)

        us_sep = per_step_us(pair)
        nhc.step_pre_force()  # the fused calls run a step's post half and the next step's pre half
        us = per_step_us(fused)
        nbytes = 220 * n
        out.append({"atoms": n, "us_per_step": round(us, 2), "launches_per_step": 1 if n <= 4096 else 3,
                    "us_per_step_separate": round(us_sep, 2), "bytes_per_step": nbytes,
                    "GBps": round(nbytes / us / 1e3, 1), "frac_of_hbm_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4)})
        log(f"NHC {n} atoms: {us:.2f} us per step fused, {us_sep:.2f} separate ({out[-1]['GBps']} GB/s)")
        del nhc
        torch.cuda.empty_cache()
    return out


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

    # the GPU path's skin rule: candidates within rc + skin (8 A), refreshed once an atom moved a
    # quarter of the skin since the last refresh, and an exact re-filter of them every step
    skin = 2.0
    state = {"ref": None}

    def forces(q):
        if state["ref"] is None or np.linalg.norm(q - state["ref"], axis=1).max() >= 0.25 * skin:
            _, wraps, wrapped = onl.wrap(q, inv, cell32)
            state.update(ref=q.copy(), wraps=wraps, cand=onl.candidates(wrapped, cell32, np.float32(64.0), 1504),
                         refreshes=state.get("refreshes", 0) + 1)
        cand = state["cand"]
        b = onl.build(q, inv, cell32, cand, state["ref"].astype(np.float32), state["wraps"], np.float32(36.0),
                      np.float32(skin + 1e-6), (1, 0, 0), int(np.minimum(cand.num_neighbors, 1504).sum()))
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
            "kind": "port", "ms_per_step": round(elapsed / steps * 1e3, 2), "cpu_model": _cpu_model(),
            "sample": f"{steps} whole MD steps (neighbour list re-filtered from skin candidates, "
                      f"{state['refreshes']} candidate refreshes, + MACE-like forward/backward + NHC) of the "
                      f"{n_atoms}-atom perovskite in PyTorch-CPU eager / NumPy, fp32 model, fp64 integrator"}


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baseline's record."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=1000)
    parser.add_argument("--warmup", type=int, default=1000,
                        help="untimed MD steps before timing (thermalisation: the edge count settles)")
    parser.add_argument("--thermalise", type=int, default=2000,
                        help="untimed equilibration steps before the warm-up (the random-init potential "
                             "keeps adding edges for ~2 000 steps from the jittered lattice)")
    parser.add_argument("--steps-small", type=int, default=2000)
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--cpu-seconds", type=float, default=15.0)
    parser.add_argument("--quick", action="store_true", help="short run (profiling): no CPU baseline, fewer steps")
    parser.add_argument("--scaling", action="store_true",
                        help="only the configs[3] size sweep (135 .. 40 000 atoms, --steps-scaling steps each)")
    parser.add_argument("--steps-scaling", type=int, default=1000)
    parser.add_argument("--ops", action="store_true",
                        help="only the configs[1] operator microbenchmark sweep (N x F), one JSON line")
    parser.add_argument("--threebody", action="store_true",
                        help="only the configs[4] three-body model (5 000 atoms, bond cutoffs 3 and 3.5 A)")
    parser.add_argument("--steps-threebody", type=int, default=500)
    parser.add_argument("--warmup-threebody", type=int, default=2000,
                        help="untimed three-body steps (the random-init potential keeps adding edges and triplets "
                             "for the first ~2 000 steps, each growth a recapture)")
    parser.add_argument("--replicas", action="store_true",
                        help="only replica batching (8 and 32 replicas of the 135-atom system)")
    parser.add_argument("--model-graph", action="store_true",
                        help="only the model_graph execution mode (MACE-like, 135 and 10 000 atoms)")
    parser.add_argument("--nhc", action="store_true",
                        help="only the NHC halves alone (135, 10 000 and 40 000 atoms)")
    parser.add_argument("--gemm-only", action="store_true",
                        help="only the configs[1] edge GEMMs at 40 000 atoms, F = 128 (the --pmc runs of the matrix cores)")
    parser.add_argument("--roofline-only", action="store_true",
                        help="only the dominant kernel at the 10 000-atom shape plus a 256 MiB copy (--pmc runs)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs the MD step on one MI355X; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is a design only in this build)", file=sys.stderr)
        return 2
    if args.steps % STEPS_PER_LAUNCH:
        print(f"--steps must be a multiple of {STEPS_PER_LAUNCH}", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    steps_small = 200 if args.quick else args.steps_small
    if args.scaling:
        print(json.dumps({"scaling": scaling_sweep(args.steps_scaling, args.warmup)}), flush=True)
        return 0
    if args.threebody:
        print(json.dumps({"threebody": threebody_bench(args.steps_threebody, args.warmup_threebody)}), flush=True)
        return 0
    if args.model_graph:
        print(json.dumps({"model_graph": model_graph_bench(200, 200)}), flush=True)
        return 0
    if args.replicas:
        print(json.dumps({"replicas_135": replica_bench(1000, 1000)}), flush=True)
        return 0
    if args.nhc:
        print(json.dumps({"nhc": nhc_bench()}), flush=True)
        return 0
    if args.ops:
        print(json.dumps({"ops_sweep": ops_sweep(), "hbm_peak_GBps": HBM_PEAK_GBPS,
                          "fp32_mfma_peak_TFLOPs": FP32_MFMA_PEAK_TFLOPS}), flush=True)
        return 0
    if args.gemm_only:
        r = hbm_ops_bench(40000, 128, gemm=True)
        print(json.dumps({k: r[k] for k in ("atoms", "edges", "F", "edge_gemm_f32", "gather_cat_edge_gemm_f32_fused",
                                              "edge_gemm_bf16")}), flush=True)
        return 0
    if args.roofline_only:
        # the run profiled with rocprofv3 --pmc for the dominant kernel's HBM traffic: it at
        # the 10 000-atom shape, then a plain 256 MiB device copy (the counters' calibration)
        md = build_md(10000, STEPS_PER_LAUNCH)
        roof = message_roofline(md)
        src = torch.empty(64 << 20, device=md.device)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"roofline": roof, "copy_bytes": src.numel() * 4}), flush=True)
        return 0

    log("10 000 atoms: capture")
    md = build_md(10000, STEPS_PER_LAUNCH)
    log("10 000 atoms: timing")
    thermalise = 200 if args.quick else args.thermalise
    t_big = time_md(md, args.steps, args.warmup, thermalise)
    ms_big = t_big / args.steps * 1e3
    stats_big = md.whole_step_stats()
    events_big = md.timed_events
    log(f"10 000 atoms: {ms_big:.3f} ms/step {events_big}")
    roof = message_roofline(md)
    del md
    torch.cuda.empty_cache()

    log("135 atoms: capture")
    md = build_md(135, STEPS_PER_LAUNCH)
    t_small = time_md(md, steps_small, args.warmup, thermalise)
    ms_small = t_small / steps_small * 1e3
    stats_small = md.whole_step_stats()
    events_small = md.timed_events
    log(f"135 atoms: {ms_small:.4f} ms/step {events_small}")
    del md
    torch.cuda.empty_cache()

    log("configs[4]: three-body model, 5 000 atoms")
    threebody = threebody_bench(200 if args.quick else args.steps_threebody,
                                200 if args.quick else args.warmup_threebody)

    log("135 atoms with a trajectory frame every 10 steps")
    frames = frames_bench(200 if args.quick else steps_small, args.warmup)
    log(f"135 atoms + frames: {frames['ms_per_step']} ms/step")

    log("replica batching")
    replicas = replica_bench(200 if args.quick else 1000, 200 if args.quick else 1000)

    log("model_graph mode")
    model_graph = model_graph_bench(50 if args.quick else 200, 50 if args.quick else 200)

    log("memory-bound operator microbenchmarks and the edge GEMM")
    seg = hbm_ops_bench(gemm=True)
    gemm_40k = {"atoms": seg["atoms"], "edges": seg["edges"], "F": seg["F"],
                "shape": [seg["edges"], 2 * seg["F"] + 8, 4 * seg["F"]],
                **{k: seg.pop(k) for k in ("edge_gemm_f32", "gather_cat_edge_gemm_f32_fused", "edge_gemm_bf16")}}
    log("NHC halves alone")
    nhc = nhc_bench()
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
                   "e_capacity": stats_big["e_capacity"],
                   "max_edges": stats_big["max_edge_count"],
                   "thermalised": f"{thermalise} untimed equilibration steps, then {args.warmup} untimed "
                                  "warm-up steps, before the timed ones"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "md_steps_per_s": round(1e3 / ms_big, 2),
        "small_system": {"atoms": 135, "ms_per_step": round(ms_small, 5), "md_steps_per_s": round(1e3 / ms_small, 1),
                         "atom_steps_per_s": round(135 / (ms_small / 1e3), 1), "steps": steps_small,
                         "e_capacity": stats_small["e_capacity"], "timed_events": events_small},
        "small_system_with_frames": frames,
        "threebody_5000": threebody,
        "model_graph": model_graph,
        "replicas_135": replicas,
        "segment_sum_GBps": seg["segment_sum"]["GBps"],
        "hbm_ops_40k": seg,
        "gemm_40k": gemm_40k,
        "nhc": nhc,
        "whole_step_stats_10k": {**{k: stats_big[k] for k in ("candidate_refreshes", "fallback_windows",
                                                              "max_edge_count", "capacity_history")},
                                 "timed_events": events_big},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
