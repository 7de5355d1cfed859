"""(a, eager) Ragged neighbour list per step for the eager and model-graph modes (HIP kernels).

Same interface as the reference's ``TensorGraphBuilder`` for the edges-only path
(fastmd/graph/gpu_graph_builder.py:935-1085): candidates at ``cutoff + 1e-6`` in
``max_neighbors`` slots per atom, grown by ``max(2 * cap, ceil(max / 16) * 16)`` when a row was
truncated (:74-85, host sync, then rebuilt: the result does not depend on the slot count), the
exact re-filter ``d < cutoff``, canonical (centre, neighbour, image) order and an isolated-atom
check; the result is a ragged ``GraphBatch`` (no padding rows).
"""
from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from fastmd_amd import _abi
from fastmd_amd.adapters.protocol import GraphBatch
from fastmd_amd.graph.neighbor_list_backend import cell_list_shape, estimate_max_neighbors
from fastmd_amd._roctx import roctx_ranged

MAX_IMAGE = 10
_NEIGHBOR_SLOT_QUANTUM = 16


def initial_max_neighbors(cutoff: float, max_neighbors: int | None) -> int:
    """gpu_graph_builder.py:74-80."""
    if max_neighbors is None:
        return int(estimate_max_neighbors(cutoff=cutoff, safety_factor=2.0))
    capacity = int(max_neighbors)
    if capacity <= 0:
        raise ValueError(f"max_neighbors must be positive, got {max_neighbors}")
    return capacity


def grown_max_neighbors(capacity: int, max_count: int) -> int:
    """gpu_graph_builder.py:83-85."""
    quantum = _NEIGHBOR_SLOT_QUANTUM
    return max(2 * capacity, -(-max_count // quantum) * quantum)


def raise_if_isolated_atoms(isolated: int) -> None:
    """fastmd/graph/validation.py:14-24."""
    if int(isolated) > 0:
        raise ValueError(f"{int(isolated)} isolated atom(s): no neighbour within the cutoff")


class TensorGraphBuilder:
    """Ragged single-system builder (see the module docstring). ``max_neighbors``: the initial
    slot count (None: the volume estimate); the grown value is kept for later builds."""

    def __init__(self, *, cell: Tensor, atomic_numbers: Tensor, pbc: Tensor | None = None,
                 atom_graph_cutoff: float = 6.0, line_graph_cutoff: float | None = 4.5,
                 device: torch.device | str = "cuda", composition: str | None = None,
                 check_isolated_atoms: bool = True, max_neighbors: int | None = None,
                 positions_dtype: torch.dtype = torch.float32) -> None:
        if line_graph_cutoff is not None:
            # the reference's default (gpu_graph_builder.py:953) asks for a 4.5 A ragged line graph
            raise NotImplementedError(
                f"TensorGraphBuilder builds the edges only: pass line_graph_cutoff=None (got {line_graph_cutoff}; "
                "the reference's default is a 4.5 A line graph). FixedCapacityGraphBuilder builds line graphs")
        if positions_dtype != torch.float32:
            raise NotImplementedError("float64 published positions are not supported")
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        _abi.load()
        if pbc is not None and not bool(torch.as_tensor(pbc).all()):
            raise NotImplementedError("non-periodic axes are not supported")
        self.cell = cell.to(device=self.device, dtype=torch.float32).contiguous()
        if tuple(self.cell.shape) != (3, 3):
            raise ValueError(f"cell must have shape (3, 3), got {tuple(self.cell.shape)}")
        self.inv_cell = torch.linalg.inv(self.cell.double().cpu()).float().to(self.device).contiguous()
        self.atomic_numbers = atomic_numbers.to(device=self.device, dtype=torch.int32)
        if self.atomic_numbers.dim() != 1:
            raise ValueError("atomic_numbers must be a 1D tensor")
        self.n_atoms = int(self.atomic_numbers.shape[0])
        self.atom_graph_cutoff = float(atom_graph_cutoff)
        self.candidate_cutoff = self.atom_graph_cutoff + 1e-6
        self.check_isolated_atoms = bool(check_isolated_atoms)
        self.max_neighbors = initial_max_neighbors(self.atom_graph_cutoff, max_neighbors)
        self.composition = composition or ""
        self.rebuilds = 0
        self._rc2 = float(np.float32(self.atom_graph_cutoff * self.atom_graph_cutoff))
        self._cand2 = float(np.float32(self.candidate_cutoff * self.candidate_cutoff))
        self._ncells, self._reach = cell_list_shape(self.cell.cpu().numpy(), self.candidate_cutoff)
        n = self.n_atoms
        dev = self.device
        ncell = self._ncells[0] * self._ncells[1] * self._ncells[2]
        self._cell_count = torch.zeros(ncell, dtype=torch.int32, device=dev)
        self._cell_start = torch.zeros(ncell + 1, dtype=torch.int32, device=dev)
        self._cell_atoms = torch.zeros(n, dtype=torch.int32, device=dev)

    @torch.no_grad()
    @roctx_ranged("neighbor_list")
    def build(self, positions: Tensor) -> GraphBatch:
        n, dev = self.n_atoms, self.device
        positions = positions.to(device=dev)
        if positions.dim() != 2 or positions.shape[1] != 3:
            raise ValueError(f"positions must have shape (N, 3), got {tuple(positions.shape)}")
        if positions.shape[0] != n:
            raise ValueError(f"positions must have the same length as atomic_numbers ({positions.shape[0]} != {n})")
        if positions.dtype not in (torch.float32, torch.float64):
            positions = positions.float()
        positions = positions.contiguous()
        is64 = 1 if positions.dtype == torch.float64 else 0
        stream = _abi.stream_handle(dev)
        f32 = dict(dtype=torch.float32, device=dev)
        i32 = dict(dtype=torch.int32, device=dev)
        frac = torch.empty((n, 3), **f32)
        wraps = torch.empty((n, 3), **i32)
        wrapped = torch.empty((n, 3), **f32)
        ref_pos = torch.empty((n, 3), **f32)
        ref_wraps = torch.empty((n, 3), **i32)
        wrap_delta = torch.empty((n, 3), **i32)
        _abi.call("fmd_nl_wrap", positions.data_ptr(), is64, self.inv_cell.data_ptr(), self.cell.data_ptr(), n,
                  frac.data_ptr(), wraps.data_ptr(), wrapped.data_ptr(), ref_pos.data_ptr(), ref_wraps.data_ptr(),
                  wrap_delta.data_ptr(), stream)
        valid = torch.empty(1, dtype=torch.uint8, device=dev)
        while True:
            bmax = self.max_neighbors
            nm = torch.empty((n, bmax), **i32)
            ns = torch.empty((n, bmax, 3), **i32)
            num = torch.empty(n, **i32)
            _abi.call("fmd_nl_candidates", wrapped.data_ptr(), frac.data_ptr(), self.cell.data_ptr(), n, self._cand2,
                      _abi.array(_abi._i32, self._ncells), _abi.array(_abi._i32, self._reach), bmax,
                      self._cell_count.data_ptr(), self._cell_start.data_ptr(), self._cell_atoms.data_ptr(),
                      nm.data_ptr(), ns.data_ptr(), num.data_ptr(), valid.data_ptr(), 0, 0, stream)
            max_count, total = torch.stack([num.max().long(), num.clamp(max=bmax).long().sum()]).tolist()
            if max_count <= bmax:
                break
            self.max_neighbors = grown_max_neighbors(bmax, max_count)
            self.rebuilds += 1
        e_cap = max(int(total), 1)
        i64 = dict(dtype=torch.int64, device=dev)
        work = torch.empty(int(_abi.load().fmd_nl_build_work_size(n)), **i64)
        counts = torch.empty(n, **i64)
        offsets = torch.empty(n + 1, **i64)
        center = torch.empty(e_cap, **i32)
        neighbor = torch.empty(e_cap, **i32)
        images = torch.empty((e_cap, 3), **i32)
        distances = torch.empty(e_cap, **f32)
        edge_index = torch.empty((e_cap, 2), **i32)
        edge_image = torch.empty((e_cap, 3), **f32)
        max_disp = torch.empty(1, **f32)
        cand_valid = torch.empty(1, dtype=torch.uint8, device=dev)
        overflow = torch.empty(1, dtype=torch.uint8, device=dev)
        isolated = torch.empty(1, **i32)
        _abi.call("fmd_nl_build", positions.data_ptr(), is64, self.inv_cell.data_ptr(), self.cell.data_ptr(), n,
                  nm.data_ptr(), ns.data_ptr(), num.data_ptr(), bmax, ref_pos.data_ptr(), ref_wraps.data_ptr(),
                  valid.data_ptr(), self._rc2, float(np.float32(1.0e-6)), 0, 0, 0, 1, 0, None, None, e_cap, work.data_ptr(),
                  frac.data_ptr(), wrap_delta.data_ptr(), wrapped.data_ptr(), counts.data_ptr(), offsets.data_ptr(),
                  center.data_ptr(), neighbor.data_ptr(), images.data_ptr(), distances.data_ptr(),
                  edge_index.data_ptr(), edge_image.data_ptr(), max_disp.data_ptr(), cand_valid.data_ptr(),
                  overflow.data_ptr(), isolated.data_ptr(), 0.0, None, None, None, None, None, None, None, 0,
                  stream)
        edges, iso = torch.stack([offsets[-1], isolated[0].long()]).tolist()
        if self.check_isolated_atoms:
            raise_if_isolated_atoms(iso)
        reverse = torch.empty(max(edges, 1), **i32)
        _abi.call("fmd_nl_reverse", center.data_ptr(), neighbor.data_ptr(), images.data_ptr(), offsets.data_ptr(), n,
                  max(edges, 1), reverse.data_ptr(), stream)
        return GraphBatch(
            positions=wrapped,
            frac_coords=frac,
            cell=self.cell,
            species=self.atomic_numbers,
            n_real=n,
            edge_index=edge_index[:edges],
            edge_image=edge_image[:edges],
            n_edges=offsets[-1:].clone(),
            cutoff=self.atom_graph_cutoff,
            padding=None,
            composition=self.composition,
            edge_offsets=offsets,
            edge_reverse=reverse[:edges],
        )

    __call__ = build
