"""The engine-owned derivative: forces of a model that returns per-atom energies only.

Same contract as the reference's ``EnergyDerivative`` (fastmd/engine/energy_derivative.py:87-140):
the leaf is a detached view of ``batch.positions`` (no copy), the energy is the FP64 sum of the
real rows' energies, one ``torch.autograd.grad`` gives F = -dE/dx, and nothing synchronizes the
host, so the whole-step runner captures it. The FP64 sum is a HIP kernel with a fixed summation
order (deterministic and free of library reductions inside a captured graph).
"""
from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd.adapters.protocol import EnergyTap, GraphBatch


class _SumF64(Function):
    @staticmethod
    def forward(ctx, x: Tensor) -> Tensor:
        x = x.detach().contiguous()
        if x.dtype not in (torch.float32, torch.float64):
            raise ValueError(f"energies must be float32 or float64, got {x.dtype}")
        out = torch.empty(1, dtype=torch.float64, device=x.device)
        _abi.call("fmd_sum_f64", x.data_ptr(), 1 if x.dtype == torch.float64 else 0, x.numel(), out.data_ptr(),
                  _abi.stream_handle())
        ctx.shape, ctx.dtype = x.shape, x.dtype
        return out.reshape(())

    @staticmethod
    def backward(ctx, g: Tensor):
        return g.to(ctx.dtype).expand(ctx.shape).contiguous()


def sum_f64(x: Tensor) -> Tensor:
    """sum(x) in float64 in a fixed order (0-dim), differentiable."""
    return _SumF64.apply(x)


def sum_f64_into(x: Tensor) -> Tensor:
    """sum(x) in float64 in the same fixed order as ``sum_f64``, as a [1] tensor, no autograd."""
    x = x.detach().contiguous()
    out = torch.empty(1, dtype=torch.float64, device=x.device)
    _abi.call("fmd_sum_f64", x.data_ptr(), 1 if x.dtype == torch.float64 else 0, x.numel(), out.data_ptr(),
              _abi.stream_handle())
    return out


def _ranges(segments, rows: int) -> list:
    """(start, count) row ranges of ``segments``: an int k (k equal contiguous slices of ``rows``,
    replicas) or a sequence of (start, count) pairs (systems of a slot union: their occupied rows)."""
    if isinstance(segments, int):
        if rows % segments:
            raise ValueError(f"{rows} rows do not split into {segments} equal segments")
        n = rows // segments
        return [(r * n, n) for r in range(segments)]
    out = [(int(a), int(c)) for a, c in segments]
    if any(a < 0 or c < 0 or a + c > rows for a, c in out):
        raise ValueError(f"segment ranges {out} exceed {rows} rows")
    return out


def sum_f64_segments(x: Tensor, segments) -> Tensor:
    """Per-segment ``sum_f64_into`` ([segments] float64) of ``segments`` (``_ranges``): each range
    summed in the order ``sum_f64`` sums a system of that size, so a replica's or a system's energy
    is bitwise its single-system energy."""
    if isinstance(segments, int) and segments == 1:
        return sum_f64_into(x)
    x = x.detach().contiguous().reshape(-1)
    ranges = _ranges(segments, x.numel())
    out = torch.empty(len(ranges), dtype=torch.float64, device=x.device)
    for r, (a, c) in enumerate(ranges):
        _abi.call("fmd_sum_f64", x[a:a + c].data_ptr(), 1 if x.dtype == torch.float64 else 0, c,
                  out[r:r + 1].data_ptr(), _abi.stream_handle())
    return out


_VIRIAL_WORK = []


def edge_stress(geo: Tensor, gvec: Tensor, n_edges: Tensor, cell: Tensor) -> Tensor:
    """The stress dE/d(strain) / V [3, 3] float32 (energy_derivative.py:110-140) from a model's
    edge geometry rows ``geo`` [e_cap, 8] (unit vector, length, ...) and the VJP's edge-vector
    gradient ``gvec`` = dE/dv [e_cap, 3] over the real rows ``n_edges``: a symmetric strain S of
    positions and cell moves every edge vector as v -> v (I + S), so dE/dS = sym(sum_e v_e gvec_e^T).
    Float64 sums in a fixed order (one HIP kernel and a one-wave finish), nothing synchronizes."""
    if not _VIRIAL_WORK:
        _VIRIAL_WORK.append(int(_abi.load().fmd_edge_virial_work_size()))
    cell = cell.detach().to(torch.float32).contiguous()
    if cell.shape != (3, 3):
        raise ValueError(f"the stress of one system needs a [3, 3] cell, got {tuple(cell.shape)}")
    work = torch.empty(_VIRIAL_WORK[0], dtype=torch.float64, device=geo.device)
    out = torch.empty(3, 3, dtype=torch.float32, device=geo.device)
    _abi.call("fmd_edge_stress_f32", geo.data_ptr(), gvec.data_ptr(), n_edges.data_ptr(), geo.shape[0],
              cell.data_ptr(), work.data_ptr(), out.data_ptr(), _abi.stream_handle())
    return out


def engine_derivative(adapter) -> "EnergyDerivative | None":
    """The derivative the runtime runs for ``adapter`` (energy_derivative.py:51-60)."""
    if hasattr(adapter, "node_energy"):
        return EnergyDerivative(adapter)
    if hasattr(adapter, "evaluate"):
        return None
    raise TypeError(f"model adapter {getattr(adapter, 'name', adapter)!r} has neither a model-owned derivative "
                    "nor an energy tap (node_energy)")


def edges_only_builder_options(adapter) -> dict:
    """Builder options beyond the defaults (energy_derivative.py:63-73): none are needed here (edges
    are always in the canonical order, which is also grouped by centre)."""
    topology = adapter.topology_spec()
    if topology.model_dtype != "float32":
        raise NotImplementedError("float64 models are not supported by the fp32 kernels")
    return {}


class EnergyDerivative:
    """``derivative(batch, inputs, task="ef", n_real=None) -> {"e": [1] f64, "f": [forces [rows, 3]]}``,
    plus ``"s": [stress [3, 3] float32, eV/A^3]`` for a task with ``"s"``."""

    stress_unit = "eV/A^3"

    def __init__(self, adapter: EnergyTap, segments: int = 1) -> None:
        self.adapter = adapter
        # replica batching: the rows are this many copies of one system; a slot union of systems:
        # (start, count) ranges of their occupied rows. "e" then holds one energy per copy or system
        # (each bitwise its single-system energy), the forces are unchanged
        self.segments = segments if not isinstance(segments, int) else int(segments)

    def extensive_energy(self, energy: Tensor, atom_counts) -> Tensor:
        return energy

    def __call__(self, batch: GraphBatch, inputs, *, task: str = "ef", n_real: int | None = None) -> dict:
        if "s" in task:
            return self._with_stress(batch, inputs, n_real)
        explicit = getattr(self.adapter, "energy_and_forces", None)
        if explicit is not None and (n_real is None or n_real == batch.positions.shape[0]):
            # the adapter's explicit VJP: the same kernels as the autograd path below without the
            # autograd seed / cast / negation launches (one graph node each per step)
            if isinstance(self.segments, int) and self.segments == 1:
                energy, forces = explicit(inputs, batch.positions, batch.cell)
            else:
                energy, forces = explicit(inputs, batch.positions, batch.cell, segments=self.segments)
            return {"e": energy, "f": [forces]}
        with torch.enable_grad():
            leaf = batch.positions.detach().requires_grad_(True)
            energies = self.adapter.node_energy(inputs, leaf, batch.cell)
            rows = energies.shape[0] if n_real is None else n_real
            if isinstance(self.segments, int) and self.segments == 1:
                energy = sum_f64(energies[:rows])
                (grad,) = torch.autograd.grad(energy, (leaf,))
                return {"e": energy.detach().reshape(1), "f": [-grad]}
            parts = torch.stack([sum_f64(energies[a:a + c]) for a, c in _ranges(self.segments, rows)])
            (grad,) = torch.autograd.grad(parts.sum(), (leaf,))
        return {"e": parts.detach(), "f": [-grad]}

    def _with_stress(self, batch: GraphBatch, inputs, n_real: int | None) -> dict:
        """``{"e", "f", "s": [stress [3, 3]]}`` of one system (energy_derivative.py:110-140): the
        adapter's ``energy_forces_stress`` forms the stress from its VJP's edge-vector gradient,
        the same kernels as its forces (which are bitwise those of the ``"ef"`` task)."""
        tap = getattr(self.adapter, "energy_forces_stress", None)
        name = getattr(self.adapter, "name", type(self.adapter).__name__)
        if tap is None:
            raise NotImplementedError(f"model {name!r} has no stress tap (energy_forces_stress)")
        if not (isinstance(self.segments, int) and self.segments == 1) or (
                batch.systems is not None and batch.systems.count > 1):
            raise NotImplementedError("stress is formed for one system per batch, not per replica or system")
        if n_real is not None and n_real != batch.positions.shape[0]:
            raise NotImplementedError("stress over a subset of the rows (n_real < rows) is not supported")
        energy, forces, stress = tap(inputs, batch.positions, batch.cell)
        return {"e": energy.reshape(1), "f": [forces], "s": [stress]}
