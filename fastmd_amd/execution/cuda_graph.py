"""Bucketed model graphs: the ``model_graph`` execution mode (one HIP graph of the model's
forward + VJP per capacity bucket, replayed each MD step).

Interface of the reference's ``BucketedGraphRunner`` (fastmd/execution/cuda_graph.py:449-860):
``run(g)`` takes a ragged ``GraphBatch`` of the eager builder (host-known row counts), copies it
into the padded workspace of the bucket that holds its demand, replays that bucket's graph and
returns ``(out, n_real)`` (``out`` valid until the next ``run``). The integrator and the ragged
build stay eager; only the model evaluation is a graph.

Buckets: ``tier(held_demand(u))`` undirected pairs (and, for a model that reads a line graph,
``tier(held_demand(t))`` triplets) with the model's capacity steps and thermal factors
(capacity_policy.py); a demand is served by the smallest cached bucket that holds it, a miss
captures a new bucket into the shared graph pool (buckets replay one at a time on one stream).

Workspaces: an edges-only model gets the ragged rows copied into fixed buffers whose tail is
the builder's far self-loop padding (``fmd_nl_pad_rows``; the reference's
``_PaddedEdgesWorkspace``, cuda_graph.py:209-293). A line-graph model gets a fixed-capacity
line-graph builder that builds the bucket's graph from the batch's positions (the pair and
triplet layouts of ``fmd_nl_line_graph``) eagerly before the replay.
"""
from __future__ import annotations

import torch
from torch import Tensor

from fastmd_amd import _abi
from fastmd_amd.adapters.protocol import GraphBatch, PaddingRule
from fastmd_amd.engine.capacity_policy import held_demand, tier
from fastmd_amd.engine.energy_derivative import engine_derivative
from fastmd_amd.execution.graph_capture import capture_graph
from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder, self_loop_padding
from fastmd_amd._roctx import roctx_ranged

_FAR_SELF_LOOPS = PaddingRule("far_self_loops")


def _demand_u(g: GraphBatch) -> int:
    return int(g.edge_index.shape[0]) // 2


def triplet_demand(g: GraphBatch, cutoff: float) -> int:
    """Triplets of a ragged build (host sync): bonds are rows whose squared float32 length is
    below the cutoff's (the builder's own test); sum s (s - 1) over the centres."""
    ei = g.edge_index.long()
    pos = g.positions.to(torch.float32)
    vec = pos.index_select(0, ei[:, 1]) + g.edge_image.to(torch.float32) @ g.cell.to(torch.float32) \
        - pos.index_select(0, ei[:, 0])
    c = torch.tensor(cutoff, dtype=torch.float32)
    short = (vec * vec).sum(1) < c * c
    s = torch.bincount(ei[short, 0], minlength=int(g.n_real))
    return int((s * (s - 1)).sum().item())


class _EdgesWorkspace:
    """Fixed [2 u_cap] edge buffers of one bucket; ``update`` copies a ragged build in and pads."""

    def __init__(self, sample: GraphBatch, u_cap: int, rule: PaddingRule, cutoff: float, device) -> None:
        n = int(sample.n_real)
        e = 2 * u_cap
        self.n, self.e_cap = n, e
        self.pad = self_loop_padding(rule, sample.cell, cutoff)[0]
        i32 = dict(dtype=torch.int32, device=device)
        self.edge_index = torch.zeros((e, 2), **i32)
        self.edge_image = torch.zeros((e, 3), dtype=torch.float32, device=device)
        self.edge_reverse = torch.full((e,), -1, **i32)
        self.edge_offsets = torch.zeros(n + 1, dtype=torch.int64, device=device)
        self.positions = torch.zeros((n, 3), dtype=torch.float32, device=device)
        self.batch = GraphBatch(positions=self.positions, frac_coords=sample.frac_coords, cell=sample.cell,
                                species=sample.species, n_real=n, edge_index=self.edge_index,
                                edge_image=self.edge_image, n_edges=self.edge_offsets[-1:], cutoff=sample.cutoff,
                                padding=rule, composition=sample.composition, edge_offsets=self.edge_offsets,
                                edge_reverse=self.edge_reverse)
        self._last = -1

    def update(self, g: GraphBatch, positions: Tensor | None = None) -> None:
        rows = int(g.edge_index.shape[0])
        if rows > self.e_cap:
            raise ValueError(f"{rows} edge rows do not fit the bucket's {self.e_cap}")
        self.edge_index[:rows].copy_(g.edge_index)
        self.edge_image[:rows].copy_(g.edge_image)
        self.edge_reverse[:rows].copy_(g.edge_reverse)
        self.edge_offsets.copy_(g.edge_offsets)
        self.positions.copy_(g.positions)
        if rows != self._last:  # the padded tail moves with the real row count
            _abi.call("fmd_nl_pad_rows", self.edge_index.data_ptr(), self.edge_image.data_ptr(),
                      self.edge_reverse.data_ptr(), rows, self.e_cap, self.n, *self.pad, _abi.stream_handle())
            self._last = rows


class _LineGraphWorkspace:
    """A fixed-capacity line-graph builder of one bucket; ``update`` builds from the batch's
    positions (eager kernels before the replay)."""

    def __init__(self, sample: GraphBatch, u_cap: int, t_cap: int, cutoff: float, triplet_cutoff: float,
                 candidate_cutoff: float, rule: PaddingRule, device) -> None:
        self.builder = FixedCapacityGraphBuilder(cell=sample.cell, atomic_numbers=sample.species, u_capacity=u_cap,
                                                 t_capacity=t_cap, atom_graph_cutoff=cutoff,
                                                 line_graph_cutoff=triplet_cutoff, candidate_cutoff=candidate_cutoff,
                                                 padding=rule, device=device)
        self.batch = self.builder.batch

    def update(self, g: GraphBatch, positions: Tensor | None = None) -> None:
        """Build from ``positions`` (the caller's coordinates, as the eager line-graph build takes
        them; default the batch's wrapped ones)."""
        from fastmd_amd.execution.whole_step_cuda_graph import FixedCapacityOverflow, _capacity_exceeded

        q = g.positions if positions is None else positions
        self.builder.refresh_candidates(q)
        _, status = self.builder.build(q, rebuild_candidates=False)
        if _capacity_exceeded(self.builder, status):
            raise FixedCapacityOverflow(int(status.edge_count.item()), int(status.triplet_count.item()))


class BucketedGraphRunner:
    """Captures one HIP graph per capacity bucket; replays the matching one
    (cuda_graph.py:449-860)."""

    def __init__(self, model, task: str = "ef", u_step: int = 512, t_step: int = 8192, n_dummy: int = 64,
                 min_pad_u: int = 256, warmup: int = 3, *, min_pad_t: int | None = None,
                 candidate_skin: float = 2.0, device: torch.device | str = "cuda") -> None:
        self.adapter = model
        self._derivative = engine_derivative(model)
        self.task = task
        self.u_step, self.t_step = int(u_step), int(t_step)
        self.min_pad_u = int(min_pad_u)
        self.min_pad_t = int(self.t_step // 2 if min_pad_t is None else min_pad_t)
        self.n_dummy = int(n_dummy)  # accepted for signature parity: the padding is far self-loops
        self.warmup = int(warmup)
        self.candidate_skin = float(candidate_skin)
        self.device = torch.device(device)
        topology = model.topology_spec()
        self.cutoff = float(topology.cutoff)
        self.triplet_cutoff = None if topology.triplet_cutoff is None else float(topology.triplet_cutoff)
        self.rule = model.padding_rule() if hasattr(model, "padding_rule") else _FAR_SELF_LOOPS
        if self.rule.kind != "far_self_loops":
            raise NotImplementedError(f"model_graph buckets pad with far self-loops, not {self.rule.kind}")
        step = model.capacity_step() if hasattr(model, "capacity_step") else None
        self._factors = (1.0, 1.0) if step is None else (float(step.u_thermal_factor), float(step.t_thermal_factor))
        self.pool = torch.cuda.graph_pool_handle()
        self.cache: dict = {}
        self.captures = 0
        self.warmup_runs = 0
        self.cache_fit_reuses = 0
        self.replays = 0
        self._n_real = None

    # ------------------------------------------------------------------ buckets
    def _key_for(self, u: int, t: int) -> tuple[int, int]:
        uf, tf = self._factors
        u_cap = tier(held_demand(u, 0, uf), self.u_step, self.min_pad_u)
        t_cap = tier(held_demand(t, 0, tf), self.t_step, self.min_pad_t) if self.triplet_cutoff is not None else 0
        return u_cap, t_cap

    def _fits(self, key, u: int, t: int) -> bool:
        # a line-graph build overflows its pairs at e_cap edges (no padding pair left)
        return (2 * u < 2 * key[0] if self.triplet_cutoff is not None else u <= key[0]) and t <= key[1]

    def _select(self, n: int, u: int, t: int):
        """(bucket, capture?) for n atoms and demand (u, t)."""
        if self.cache and n != self._n_real:
            raise ValueError(f"the runner replays {self._n_real} atoms, got {n}")
        fitting = [k for k in self.cache if self._fits(k, u, t)]
        if fitting:
            key = min(fitting)
            if key != self._key_for(u, t):
                self.cache_fit_reuses += 1
            return key, False
        return self._key_for(u, t), True

    def _capture(self, key, sample: GraphBatch, positions: Tensor | None = None) -> dict:
        if self.triplet_cutoff is None:
            ws = _EdgesWorkspace(sample, key[0], self.rule, self.cutoff, self.device)
        else:
            ws = _LineGraphWorkspace(sample, key[0], key[1], self.cutoff, self.triplet_cutoff,
                                     self.cutoff + self.candidate_skin, self.rule, self.device)
        ws.update(sample, positions)
        inputs = self.adapter.prepare(ws.batch)  # host checks, outside the capture
        n = int(sample.n_real)
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(self.warmup):
                self._derivative(ws.batch, inputs, task=self.task, n_real=n)
                self.warmup_runs += 1
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with capture_graph(graph, pool=self.pool, name="model_graph_capture"):
            out = self._derivative(ws.batch, inputs, task=self.task, n_real=n)
        entry = {"graph": graph, "workspace": ws, "inputs": inputs, "out": out, "n_real": n}
        self.cache[key] = entry
        self.captures += 1
        self._n_real = n
        return entry

    def captures_next(self, g: GraphBatch) -> bool:
        """True if ``run(g)`` would capture (run model code), not only replay."""
        n, u, t = self._demand(g)
        return self._select(n, u, t)[1]

    def _demand(self, g: GraphBatch) -> tuple[int, int, int]:
        t = triplet_demand(g, self.triplet_cutoff) if self.triplet_cutoff is not None else 0
        return int(g.n_real), _demand_u(g), t

    @roctx_ranged("model_graph_run")
    def run(self, g: GraphBatch, positions: Tensor | None = None):
        """(out, n_real) of the model on the ragged build ``g``; ``out`` is valid until the next run.
        ``positions``: the coordinates ``g`` was built from, for a line-graph model's own build
        (default: the batch's wrapped coordinates)."""
        from fastmd_amd.execution.whole_step_cuda_graph import FixedCapacityOverflow

        n, u, t = self._demand(g)
        key, capture = self._select(n, u, t)
        entry = None
        while entry is None:
            try:
                if capture:
                    entry = self._capture(key, g, positions)
                else:
                    entry = self.cache[key]
                    entry["workspace"].update(g, positions)
            except FixedCapacityOverflow as overflow:
                # a line-graph bucket's own build counted more than the ragged estimate: the next
                # bucket up that holds what it counted
                entry, capture = None, True
                u = max(u, (overflow.edge_count + 2) // 2)
                t = max(t, overflow.triplet_count)
                key = self._key_for(u, t)
                self.cache.pop(key, None)
        entry["graph"].replay()
        self.replays += 1
        return entry["out"], entry["n_real"]

    def stats(self) -> dict:
        return {"captures": self.captures, "warmup_runs": self.warmup_runs, "cache_fit_reuses": self.cache_fit_reuses,
                "replays": self.replays, "cached_buckets": [list(k) for k in sorted(self.cache)],
                "shared_graph_pool": True}
