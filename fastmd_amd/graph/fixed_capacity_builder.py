"""(a) Capture-safe fixed-capacity neighbour list for GPU-resident MD (HIP kernels).

Same interface as the reference's ``FixedCapacityGraphBuilder``
(fastmd/graph/fixed_capacity_builder.py:1030-2366) for the edges-only single-system path:
persistent buffers published as a ``GraphBatch``, a rare eager candidate refresh (cell list
within ``candidate_cutoff = cutoff + skin``) and a per-step exact re-filter ``build`` that is
a fixed sequence of kernels with device-side status flags (no host sync, capturable).

MI355X design: the candidate rows are written sorted by (neighbour, shift) at refresh, so the
per-step rows come out in the canonical (centre, neighbour, image) order directly (the
reference's per-build ``torch.sort`` of e_cap keys, :1968-1999, is gone); a build is one
fused single-workgroup kernel up to 1024 atoms, three kernels beyond (count, scan,
materialize+pad), plus the reverse-edge index that the deterministic VJPs use.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np
import torch
from torch import Tensor

from fastmd_amd import _abi
from fastmd_amd._device import require_cuda
from fastmd_amd._roctx import roctx_ranged
from fastmd_amd.adapters.protocol import GraphBatch, PaddingRule
from fastmd_amd.graph.neighbor_list_backend import (NeighborOverflowError, cell_list_shape,
                                                    estimate_max_neighbors)

_FAR_SELF_LOOPS = PaddingRule("far_self_loops")
_SINK_PADDING = PaddingRule("sink_atoms")  # the reference's default (fixed_capacity_builder.py:937,1109)


@dataclass
class FixedCapacityGraphStatus:
    """Device-side status of one build (fixed_capacity_builder.py:756-767)."""

    edge_count: Tensor
    triplet_count: Tensor
    overflow: Tensor
    invalid_pairs: Tensor
    candidate_valid: Tensor
    max_displacement: Tensor
    isolated_atom_count: Tensor
    candidate_capacity_valid: Tensor | None = None

    @property
    def undirected_count(self) -> Tensor:
        return self.edge_count // 2


def fixed_capacity_exceeded(status, builder) -> Tensor:
    """Device predicate: the real graph does not fit (fixed_capacity_builder.py:796-814). An
    edges-only builder fits up to ``e_capacity`` inclusive; with a line graph, equality is an
    overflow too."""
    if getattr(builder, "edges_only", False):
        return (status.edge_count[0] > builder.e_capacity) | status.invalid_pairs[0]
    return ((status.edge_count[0] >= builder.e_capacity) | (status.triplet_count[0] > builder.t_capacity)
            | status.invalid_pairs[0])


def self_loop_padding(padding: PaddingRule, cell: Tensor, cutoff: float):
    """(integer image, length, override vector) of the padded self-loops
    (fixed_capacity_builder.py:1004-1027). Host only."""
    if padding.kind == "exact_rc_loops":
        vector = tuple(map(float, padding.pad_vector or (cutoff, 0.0, 0.0)))
        length = float(torch.linalg.vector_norm(torch.tensor(vector, dtype=torch.float32)))
        if not length >= float(torch.tensor(cutoff, dtype=torch.float32)) or length == 0.0:
            raise ValueError(f"exact_rc_loops: pad_vector {vector} is shorter than the cutoff {cutoff}")
        return (0, 0, 0), length, vector
    if padding.kind != "far_self_loops":
        raise ValueError(f"{padding.kind} padding has no self-loops")
    lengths = cell.detach().cpu().double().norm(dim=1)
    axis = int(torch.argmax(lengths))
    longest = float(lengths[axis])
    if not longest > 0.0:
        raise ValueError("far self-loop padding needs a cell with a nonzero lattice vector")
    multiple = max(1, math.ceil(max(padding.min_length, 2.0 * cutoff) / longest))
    image = [0, 0, 0]
    image[axis] = multiple
    return (image[0], image[1], image[2]), multiple * longest, None


def _batch_itself(batch: GraphBatch) -> GraphBatch:
    return batch


# Candidate-list state a ``candidates_from`` builder shares with its source
# (fixed_capacity_builder.py:665-675): the cell list, the candidates and the refresh's reference.
_CANDIDATE_STATE = ("_cell_count", "_cell_start", "_cell_atoms", "neighbor_matrix", "neighbor_shifts",
                    "num_neighbors", "reference_positions", "reference_wraps", "wrap_delta", "_wraps",
                    "_wrapped_refresh", "_candidate_capacity_valid", "atom_order")


def morton_order(frac: Tensor, system_of: Tensor | None = None) -> Tensor:
    """The atoms sorted along a Morton (Z-order) curve of their fractional coordinates (10 bits per
    axis; a union's system index above them), int32 on the device, without a host sync: atoms
    near in the order are near in space, so kernels that take one atom per wave in this order
    gather their neighbours' rows from the same L2."""
    q = (frac.clamp(0.0, 1.0 - 1e-7) * 1024.0).to(torch.int64)

    def spread(v: Tensor) -> Tensor:  # the 10 bits of v at every third position
        v = (v | (v << 16)) & 0x030000FF
        v = (v | (v << 8)) & 0x0300F00F
        v = (v | (v << 4)) & 0x030C30C3
        return (v | (v << 2)) & 0x09249249

    code = spread(q[:, 0]) | (spread(q[:, 1]) << 1) | (spread(q[:, 2]) << 2)
    if system_of is not None:
        code = code | (system_of.to(torch.int64) << 30)
    return torch.argsort(code, stable=True).to(torch.int32)


class FixedCapacityGraphBuilder:
    """Single-system fixed-capacity builder (see the module docstring): with the three-body line
    graph (undirected pairs, short-bond lists and triplet rows, fmd_nl_line_graph, published as
    ``batch.pair_d2u`` / ``pair_u2d`` / ``triplets``), or edges only with
    ``line_graph_cutoff=None`` and ``t_capacity=0``.

    The defaults are the reference's (fixed_capacity_builder.py:1047-1070,1109): ``t_capacity``
    has none, ``line_graph_cutoff=4.5`` and ``padding=None`` means sink atoms. Padding
    (``padding``, protocol.py:68-119): sink atoms (``n_dummy`` sink rows after the real ones at
    the origin, atomic number 1; padded rows, and with a line graph padded triplets, sit on them),
    far self-loops (what this build's HIP models take) or exact-cutoff loops (edges only: image 0
    and ``batch.edge_vec_override``). Unsupported reference options (ghost rows, float64 published
    positions) raise ``NotImplementedError``. ``sorted_edges=False`` is accepted: the rows are
    always in the canonical order, which is also grouped by centre."""

    def __init__(self, *, cell: Tensor, atomic_numbers: Tensor, u_capacity: int, t_capacity: int,
                 pbc: Tensor | None = None, atom_graph_cutoff: float = 6.0, line_graph_cutoff: float | None = 4.5,
                 n_dummy: int = 64, device: torch.device | str = "cuda", composition: str | None = None,
                 candidate_cutoff: float | None = None, ghosts=None, minimum_image: bool = False,
                 candidates_from=None, padding: PaddingRule | None = None,
                 prepare: Callable[[GraphBatch], Any] | None = None, positions_dtype: torch.dtype = torch.float32,
                 sorted_edges: bool = True, max_neighbor_count: Tensor | None = None,
                 publish_positions: bool = False, system_size: int = 0) -> None:
        line_graph = line_graph_cutoff is not None
        if line_graph and (t_capacity <= 0 or not 0.0 < float(line_graph_cutoff) <= float(atom_graph_cutoff)):
            raise ValueError("a line-graph builder needs t_capacity > 0 and 0 < line_graph_cutoff <= the atom cutoff")
        if not line_graph and t_capacity != 0:
            raise ValueError("t_capacity needs a line_graph_cutoff")
        if ghosts is not None:
            raise NotImplementedError("ghost rows are not supported")
        if positions_dtype != torch.float32:
            raise NotImplementedError("float64 published positions are not supported")
        padding = _SINK_PADDING if padding is None else padding
        if line_graph and padding.kind == "exact_rc_loops":
            raise ValueError("a builder with a line graph pads with sink atoms, or a single-system builder "
                             "with far self-loops (padded triplets need padded pairs)")
        if padding.kind == "sink_atoms" and int(n_dummy) <= 0:
            raise ValueError("sink padding needs n_dummy > 0")
        if padding.kind == "sink_atoms" and system_size:
            raise NotImplementedError("replica unions pad with far self-loops")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the fixed-capacity builder runs on the GPU")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        _abi.load()
        if pbc is not None and not bool(torch.as_tensor(pbc).all()):
            raise NotImplementedError("non-periodic axes are not supported")
        self.edges_only = not line_graph
        # replica batching: the atoms are copies of one system of this many atoms, side by side;
        # no edge joins two copies (0: one system)
        self.system_size = int(system_size)
        self.padding = padding
        self.sorted_edges = True
        self.max_neighbor_count = max_neighbor_count
        self.cell = cell.to(device=self.device, dtype=torch.float32).contiguous()
        self.inv_cell = torch.linalg.inv(self.cell.double().cpu()).float().to(self.device).contiguous()
        self.atomic_numbers_real = atomic_numbers.to(device=self.device, dtype=torch.int32)
        self.n_real = int(self.atomic_numbers_real.shape[0])
        if self.n_real <= 0:
            raise ValueError("a builder needs at least one atom")
        # sink rows exist only for sink padding (fixed_capacity_builder.py:1144-1145)
        self.n_dummy = int(n_dummy) if padding.kind == "sink_atoms" else 0
        self.u_capacity = int(u_capacity)
        if self.u_capacity <= 0:
            raise ValueError("a builder needs u_capacity > 0")
        self.e_capacity = 2 * self.u_capacity
        self.t_capacity = int(t_capacity) if line_graph else 0
        self.atom_graph_cutoff = float(atom_graph_cutoff)
        self.line_graph_cutoff = float(line_graph_cutoff) if line_graph else None
        # the short-bond decision d2 < float32(cutoff^2), on the edge decision's own d2
        self._line2 = float(np.float32(self.line_graph_cutoff * self.line_graph_cutoff)) if line_graph else 0.0
        self.candidate_cutoff = float(candidate_cutoff or (self.atom_graph_cutoff + 1.0e-6))
        if self.candidate_cutoff < self.atom_graph_cutoff:
            raise ValueError("candidate_cutoff must not be below the pair cutoff")
        self.skin = self.candidate_cutoff - self.atom_graph_cutoff
        self.composition = composition or ""
        self.buffer_max = int(estimate_max_neighbors(cutoff=self.candidate_cutoff, safety_factor=2.0))
        self._rc2 = float(np.float32(self.atom_graph_cutoff * self.atom_graph_cutoff))
        self._cand2 = float(np.float32(self.candidate_cutoff * self.candidate_cutoff))
        self._skin_limit = float(np.float32(self.skin + 1.0e-6))
        # (image, length, override vector) of self-loop padding; None for sink padding
        self._pad_loop = (None if padding.kind == "sink_atoms"
                          else self_loop_padding(padding, self.cell, self.atom_graph_cutoff))
        self._ncells, self._reach = cell_list_shape(self.cell.cpu().numpy(), self.candidate_cutoff)
        # minimum_image: the caller may hand in coordinates wrapped by any lattice vector since the
        # refresh (ASE's atoms.wrap()); the skin test and the wrap delta remove the jump
        # (fixed_capacity_builder.py:1071-1074,2233-2245)
        self.minimum_image = bool(minimum_image)
        # several systems in one union (the slot-union builder sets these): the system of each row
        # and each system's far self-loop image; None for one system
        self._system_of = None
        self._pad_images = None
        n, dev = self.n_real, self.device
        i32 = dict(dtype=torch.int32, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        i64 = dict(dtype=torch.int64, device=dev)
        u8 = dict(dtype=torch.uint8, device=dev)
        # candidates_from: read (and refresh) another builder's candidate list of the same system,
        # with capacities of its own (fixed_capacity_builder.py:1075-1078,1228-1239)
        self._candidate_source = None
        if candidates_from is not None:
            source = candidates_from._candidate_owner
            if (source.device != self.device or source.n_real != self.n_real
                    or source.candidate_cutoff != self.candidate_cutoff or source.minimum_image != self.minimum_image
                    or source.system_size != self.system_size or not torch.equal(source.cell, self.cell)):
                raise ValueError("candidates_from must be a single-system builder of the same system, "
                                 "cell, pbc, candidate cutoff and minimum_image setting")
            self._candidate_source = source
            for name in _CANDIDATE_STATE:
                setattr(self, name, getattr(source, name))
        else:
            ncell = self._ncells[0] * self._ncells[1] * self._ncells[2]
            self._cell_count = torch.zeros(ncell, **i32)
            self._cell_start = torch.zeros(ncell + 1, **i32)
            self._cell_atoms = torch.zeros(n, **i32)
            self.neighbor_matrix = torch.full((n, self.buffer_max), n, **i32)
            self.neighbor_shifts = torch.zeros((n, self.buffer_max, 3), **i32)
            self.num_neighbors = torch.zeros(n, **i32)
            self.reference_positions = torch.zeros((n, 3), **f32)
            self.reference_wraps = torch.zeros((n, 3), **i32)
            self.wrap_delta = torch.zeros((n, 3), **i32)
            self._wraps = torch.zeros((n, 3), **i32)
            self._wrapped_refresh = torch.zeros((n, 3), **f32)
            self._candidate_capacity_valid = torch.zeros(1, **u8)
            self._candidate_initialized = False
            self.atom_order = torch.arange(n, **i32)
        # real rows, then the sink rows (kept at the origin)
        self.frac_coords = torch.zeros((n + self.n_dummy, 3), **f32)
        self.edge_counts = torch.zeros(n, **i64)
        self.edge_offsets = torch.zeros(n + 1, **i64)
        self.pair_offsets = torch.zeros(1, **i64)
        e = self.e_capacity
        self.center = torch.zeros(e, **i32)
        self.neighbor = torch.zeros(e, **i32)
        self.images = torch.zeros((e, 3), **i32)
        self.distances = torch.zeros(e, **f32)
        self.edge_reverse = torch.full((e,), -1, **i32)
        self._work = torch.zeros(int(_abi.load().fmd_nl_build_work_size(n)), **i64)
        self._max_displacement = torch.zeros(1, **f32)
        self._candidate_valid = torch.zeros(1, **u8)
        self._overflow = torch.zeros(1, **u8)
        self._isolated_atom_count = torch.zeros(1, **i32)
        self._invalid_pairs = torch.zeros(1, dtype=torch.bool, device=dev)
        self.short_flags = self.directed2undirected = self.undirected2directed = self.line_graph = None
        self.short_counts = self.short_offsets = self.short_edge_matrix = None
        self.edge_triplet_offsets = self.bond_rows = self.second_perm = None
        if line_graph:
            self.short_flags = torch.zeros(e, **u8)
            self.directed2undirected = torch.zeros(e, **i32)
            self.undirected2directed = torch.zeros(self.u_capacity, **i32)
            self.short_counts = torch.zeros(n, **i64)
            self.short_offsets = torch.zeros(n + 1, **i64)
            self.short_edge_matrix = torch.zeros((n, self.buffer_max), **i32)
            self.pair_offsets = torch.zeros(n + 1, **i64)
            self.line_graph = torch.zeros((self.t_capacity, 5), **i32)
            self.edge_triplet_offsets = torch.zeros(e + 1, **i64)  # angle -> bond CSR over the rows
            self.bond_rows = torch.full((e,), -1, **i32)  # short rows in (atom, rank) order
            # with edge_triplet_offsets: the triplets of each row as their second bond
            self.second_perm = torch.full((self.t_capacity,), -1, **i32)
            self._lg_work = torch.zeros(int(_abi.load().fmd_nl_line_graph_work_size(n, e)), **i64)
        self.positions = torch.zeros((n + self.n_dummy, 3), **f32)
        self.edge_vec_override = (torch.zeros((e, 3), **f32) if padding.kind == "exact_rc_loops" else None)
        species = self.atomic_numbers_real
        if self.n_dummy:
            species = torch.cat([species, torch.ones(self.n_dummy, **i32)])
        self.batch = GraphBatch(
            positions=self.positions,
            frac_coords=self.frac_coords,
            cell=self.cell,
            species=species,
            n_real=n,
            edge_index=torch.zeros((e, 2), **i32),
            edge_image=torch.zeros((e, 3), **f32),
            n_edges=self.edge_offsets[-1:],
            cutoff=self.atom_graph_cutoff,
            padding=padding,
            edge_vec_override=self.edge_vec_override,
            composition=self.composition,
            edge_offsets=self.edge_offsets,
            edge_reverse=self.edge_reverse,
            triplet_cutoff=self.line_graph_cutoff,
            pair_d2u=self.directed2undirected,
            pair_u2d=self.undirected2directed,
            triplets=self.line_graph,
            line=self._line_layout(),
            atom_order=self.atom_order,
            max_system_rows=self.system_size or n,
        )
        self.graph = (prepare or _batch_itself)(self.batch)

    def _line_layout(self):
        if self.line_graph is None:
            return None
        from fastmd_amd.ops.threebody import LineGraph

        return LineGraph.from_builder(self)

    # ------------------------------------------------------------------ candidates
    @property
    def _candidate_owner(self) -> "FixedCapacityGraphBuilder":
        """The builder whose candidate list this one reads (itself unless ``candidates_from``)."""
        return self._candidate_source or self

    def _stream(self) -> int:
        return _abi.stream_handle(self.device)

    @torch.no_grad()
    @roctx_ranged("fixed_capacity_refresh_candidates")
    def refresh_candidates(self, positions: Tensor) -> None:
        """Refresh the cell-list candidates from ``positions`` (eager, rare path): the reference
        positions and wraps are reset and the wrap delta zeroed (fixed_capacity_builder.py:1674-1685)."""
        positions = self._positions_arg(positions)
        is64 = 1 if positions.dtype == torch.float64 else 0
        n = self.n_real
        _abi.call("fmd_nl_wrap", positions.data_ptr(), is64, self.inv_cell.data_ptr(), self.cell.data_ptr(), n,
                  self.frac_coords.data_ptr(), self._wraps.data_ptr(), self._wrapped_refresh.data_ptr(),
                  self.reference_positions.data_ptr(), self.reference_wraps.data_ptr(),
                  self.wrap_delta.data_ptr(), self._stream())
        _abi.call("fmd_nl_candidates", self._wrapped_refresh.data_ptr(), self.frac_coords.data_ptr(),
                  self.cell.data_ptr(), n, self._cand2, _abi.array(_abi._i32, self._ncells),
                  _abi.array(_abi._i32, self._reach), self.buffer_max, self._cell_count.data_ptr(),
                  self._cell_start.data_ptr(), self._cell_atoms.data_ptr(), self.neighbor_matrix.data_ptr(),
                  self.neighbor_shifts.data_ptr(), self.num_neighbors.data_ptr(),
                  self._candidate_capacity_valid.data_ptr(), self.system_size, 0, self._stream())
        self.atom_order.copy_(morton_order(self.frac_coords[:n]))
        self._candidate_owner._candidate_initialized = True

    def assert_candidate_capacity(self) -> None:
        """Raise (host sync) if a candidate row was truncated (fixed_capacity_builder.py:1665-1672)."""
        if bool(self._candidate_capacity_valid.item()):
            return
        raise NeighborOverflowError(self.buffer_max, int(self.num_neighbors.max().item()))

    def _positions_arg(self, positions: Tensor) -> Tensor:
        if positions.shape != (self.n_real, 3):
            raise ValueError(f"positions must have shape {(self.n_real, 3)}, got {tuple(positions.shape)}")
        if positions.device != self.device:
            positions = positions.to(self.device)
        if positions.dtype not in (torch.float32, torch.float64):
            positions = positions.to(torch.float32)
        return positions.contiguous()

    # ------------------------------------------------------------------ build
    @torch.no_grad()
    @roctx_ranged("fixed_capacity_graph_build")
    def build(self, positions: Tensor, *, rebuild_candidates: bool = True, predicate=None, window: dict | None = None):
        """Build into the persistent buffers; returns ``(prepare(batch), status)``
        (fixed_capacity_builder.py:2180-2298). ``positions`` float32 or float64 [N, 3]. ``window``
        (the keyword arguments of ``accumulate_window``): this build's status is also folded into
        a whole-step window's flags, by the build's own launch for an edges-only build."""
        if predicate is not None:
            raise NotImplementedError("caller predicates belong to ghost-row builders")
        fold = None
        if window is not None:
            self._check_window(**window)
            if self.line_graph is None:
                fold = window
        positions = self._positions_arg(positions)
        if rebuild_candidates:
            self.refresh_candidates(positions)
        elif not self._candidate_owner._candidate_initialized:
            raise RuntimeError("refresh_candidates must run before candidate reuse")
        is64 = 1 if positions.dtype == torch.float64 else 0
        image = self._pad_image
        _abi.call("fmd_nl_build", positions.data_ptr(), is64, self.inv_cell.data_ptr(), self.cell.data_ptr(),
                  self.n_real, self.neighbor_matrix.data_ptr(), self.neighbor_shifts.data_ptr(),
                  self.num_neighbors.data_ptr(), self.buffer_max, self.reference_positions.data_ptr(),
                  self.reference_wraps.data_ptr(), self._candidate_capacity_valid.data_ptr(), self._rc2,
                  self._skin_limit, 1 if self.minimum_image else 0, image[0], image[1], image[2], self.n_dummy,
                  _abi.ptr(self._system_of), _abi.ptr(self._pad_images), self.e_capacity, self._work.data_ptr(),
                  self.frac_coords.data_ptr(), self.wrap_delta.data_ptr(), self.positions.data_ptr(),
                  self.edge_counts.data_ptr(), self.edge_offsets.data_ptr(), self.center.data_ptr(),
                  self.neighbor.data_ptr(), self.images.data_ptr(), self.distances.data_ptr(),
                  self.batch.edge_index.data_ptr(), self.batch.edge_image.data_ptr(),
                  self._max_displacement.data_ptr(), self._candidate_valid.data_ptr(), self._overflow.data_ptr(),
                  self._isolated_atom_count.data_ptr(), self._line2, _abi.ptr(self.short_flags),
                  self.edge_reverse.data_ptr(), *self._window_ptrs(fold), self._stream())
        if not self.edges_only:
            # pairs, short-bond lists and triplets; the overflow flag becomes the line-graph rule
            # (edges >= e_capacity | triplets > t_capacity | invalid pairs | invalid candidates)
            _abi.call("fmd_nl_line_graph", self.center.data_ptr(), self.edge_reverse.data_ptr(),
                      self.short_flags.data_ptr(), self.edge_offsets.data_ptr(), self._candidate_valid.data_ptr(),
                      self.n_real, self.e_capacity, self.u_capacity, self.t_capacity, self.buffer_max,
                      self._lg_work.data_ptr(), self.directed2undirected.data_ptr(),
                      self.undirected2directed.data_ptr(), self._invalid_pairs.data_ptr(),
                      self.short_counts.data_ptr(), self.short_offsets.data_ptr(),
                      self.short_edge_matrix.data_ptr(), self.pair_offsets.data_ptr(), self._overflow.data_ptr(),
                      self.line_graph.data_ptr(), self.edge_triplet_offsets.data_ptr(), self.bond_rows.data_ptr(),
                      self.second_perm.data_ptr(), self.n_dummy, self._stream())
            # an overflowed build publishes the all-padding edge rows (_substitute_overflow_topology)
            _abi.call("fmd_nl_overflow_rows", self._overflow.data_ptr(), self.n_real, self.e_capacity, self.n_dummy,
                      image[0], image[1], image[2], self.center.data_ptr(), self.neighbor.data_ptr(),
                      self.images.data_ptr(), self.batch.edge_index.data_ptr(), self.batch.edge_image.data_ptr(),
                      self._stream())
        if self.edge_vec_override is not None:
            v = self._pad_loop[2]
            _abi.call("fmd_nl_pad_override", self.edge_offsets[-1:].data_ptr(), self.e_capacity, v[0], v[1], v[2],
                      self.edge_vec_override.data_ptr(), self._stream())
        if self.max_neighbor_count is not None:
            torch.maximum(self.max_neighbor_count, self.edge_counts.max().reshape(1), out=self.max_neighbor_count)
        if window is not None and fold is None:
            self.accumulate_window(self.status, **window)
        return self.graph, self.status

    @staticmethod
    def _window_ptrs(window: dict | None) -> tuple:
        """fmd_nl_build's window arguments (all null: no fold)."""
        if window is None:
            return (None, None, None, None, None, 0)
        stats = window.get("stats")
        return (window["window_overflow"].data_ptr(), window["window_capacity_overflow"].data_ptr(),
                window["window_max_edges"].data_ptr(), window["window_max_isolated"].data_ptr(),
                None if stats is None else stats.data_ptr(), 1 if window["check_isolated"] else 0)

    @staticmethod
    def _check_window(*, window_overflow: Tensor, window_capacity_overflow: Tensor, window_max_edges: Tensor,
                      window_max_isolated: Tensor, check_isolated: bool, stats: Tensor | None = None,
                      window_max_triplets: Tensor | None = None) -> None:
        if window_max_triplets is not None and window_max_triplets.dtype != torch.int64:
            raise ValueError("window_max_triplets must be int64")
        if stats is not None and (stats.dtype != torch.float64 or stats.numel() < 7):
            raise ValueError("stats must be a float64 tensor of at least 7 entries")
        for t, dt in ((window_overflow, torch.uint8), (window_capacity_overflow, torch.uint8),
                      (window_max_edges, torch.int64), (window_max_isolated, torch.int32)):
            if t.dtype != dt:
                raise ValueError(f"window flag dtype {t.dtype}, expected {dt}")

    @property
    def _pad_image(self) -> tuple[int, int, int]:
        """The self-loop padding image (unused by sink padding)."""
        return (0, 0, 0) if self._pad_loop is None else self._pad_loop[0]

    @property
    def status(self) -> FixedCapacityGraphStatus:
        return FixedCapacityGraphStatus(
            edge_count=self.edge_offsets[-1:],
            triplet_count=self.pair_offsets[-1:],
            overflow=self._overflow,
            invalid_pairs=self._invalid_pairs,
            candidate_valid=self._candidate_valid,
            max_displacement=self._max_displacement,
            isolated_atom_count=self._isolated_atom_count,
            candidate_capacity_valid=self._candidate_capacity_valid,
        )

    def accumulate_window(self, status: FixedCapacityGraphStatus, *, window_overflow: Tensor,
                          window_capacity_overflow: Tensor, window_max_edges: Tensor, window_max_isolated: Tensor,
                          check_isolated: bool, stats: Tensor | None = None,
                          window_max_triplets: Tensor | None = None) -> None:
        """Fold one build's status into a whole-step window's flags in one kernel
        (fixed_capacity_builder.py:2300-2312, 430-455). Flags are uint8 [1]; ``stats`` (float64 [7])
        receives the window's statistics after this build. A line-graph build also folds its
        triplet count (capacity overflow above t_capacity, pairs full at e_capacity edges) and
        its invalid-pair flag."""
        self._check_window(window_overflow=window_overflow, window_capacity_overflow=window_capacity_overflow,
                           window_max_edges=window_max_edges, window_max_isolated=window_max_isolated,
                           check_isolated=check_isolated, stats=stats, window_max_triplets=window_max_triplets)
        line = self.line_graph is not None
        _abi.call("fmd_nl_window_flags", status.edge_count.data_ptr(),
                  status.invalid_pairs.data_ptr() if line else None, status.overflow.data_ptr(),
                  status.isolated_atom_count.data_ptr(), self.e_capacity, 1 if check_isolated else 0,
                  window_overflow.data_ptr(), window_capacity_overflow.data_ptr(), window_max_edges.data_ptr(),
                  window_max_isolated.data_ptr(), status.max_displacement.data_ptr(),
                  None if stats is None else stats.data_ptr(), status.triplet_count.data_ptr() if line else None,
                  self.t_capacity, _abi.ptr(window_max_triplets) if line else None, self._stream())

    # ------------------------------------------------------------------ host views (tests, eager)
    def real_edges(self) -> tuple[Tensor, Tensor, Tensor]:
        """(center, neighbor, images) of the real rows (host sync)."""
        count = min(int(self.edge_offsets[-1].item()), self.e_capacity)
        return self.center[:count], self.neighbor[:count], self.images[:count]
