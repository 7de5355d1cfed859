"""Three-body Fourier angle basis on the GPU (HIP kernels), forward and deterministic VJP.

``threebody_fourier_basis`` keeps the reference's signature and meaning
(``fastmd/models/matris/op/triton_threebody_fourier.py:273-298``): for row t,
``c = (u[target[t]] . u[source[t]]) (1 - 1e-6)``, ``theta = acos(c)``,
``out[t] = [1/sqrt(2), sin(theta f), cos(theta f)] / scale`` with 1 + 2F columns, frozen
frequencies, gradient for ``unit_vec`` only. Where the reference's backward adds with float
atomics (:99-166), or with ordered ``index_add_`` in its deterministic mode (:169-181), this
one forms the per-row terms in one kernel and sums them per vector row through a CSR in a
fixed order (target terms, then source terms, each in row order), so repeated runs agree
bit for bit.

``threebody_fourier_line`` takes the triplets straight from a fixed-capacity line graph
(``fmd_nl_line_graph``): one wave per atom forms its ordered bond pairs from the short-bond
lists, and its VJP sums each short bond's terms in triplet order inside the atom's wave (no
index arrays, sort or atomics). Padding triplets (rows past the real count, indexing the
padding pairs) are written by the forward; the VJP covers the real triplets, so the padding
rows' gradient is zero, which is exact whenever nothing downstream reads padding triplets
(their gradient is then zero); the general form gives the padding terms when needed. An
overflowed build (its flag set) has only padding rows: all read from ``line_graph``, zero VJP.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd._device import require_cuda, rows_view, stream
from fastmd_amd.ops.csr_segment_sum import csr_from_segment, segment_sum_csr

MAX_FREQ = 16


def _freqs(freqs: Tensor, device) -> Tensor:
    f = freqs.detach().to(device=device, dtype=torch.float32).contiguous().reshape(-1)
    if not 1 <= f.numel() <= MAX_FREQ:
        raise ValueError(f"between 1 and {MAX_FREQ} frequencies, got {f.numel()}")
    return f


def _unit(unit_vec: Tensor) -> tuple[Tensor, int]:
    if unit_vec.dim() != 2 or unit_vec.shape[1] != 3:
        raise ValueError(f"expected unit_vec [E, 3], got {tuple(unit_vec.shape)}")
    if unit_vec.dtype != torch.float32:
        raise ValueError(f"unit_vec must be float32, got {unit_vec.dtype}")
    return rows_view(unit_vec)


def _index(index: Tensor, rows: int, name: str) -> Tensor:
    if index.dim() != 1 or index.numel() != rows:
        raise ValueError(f"{name} must be 1-D with {rows} rows, got {tuple(index.shape)}")
    return index.to(torch.int32).contiguous() if index.dtype != torch.int32 or not index.is_contiguous() else index


def _check_range(index: Tensor, n_vec: int, name: str) -> None:
    if index.numel() and (int(index.min()) < 0 or int(index.max()) >= n_vec):
        raise IndexError(f"{name} out of range for {n_vec} vectors")


class _FourierBasis(Function):
    @staticmethod
    def forward(ctx, unit_vec, target_index, source_index, freqs, scale, check_range):
        device = require_cuda(unit_vec, target_index, source_index)
        u, ld = _unit(unit_vec)
        rows = int(target_index.numel())
        tgt = _index(target_index, rows, "target_index")
        src = _index(source_index, rows, "source_index")
        if check_range:
            _check_range(tgt, u.shape[0], "target_index")
            _check_range(src, u.shape[0], "source_index")
        f = _freqs(freqs, device)
        out = torch.empty((rows, 1 + 2 * f.numel()), dtype=torch.float32, device=device)
        _abi.call("fmd_threebody_fourier_f32", u.data_ptr(), ld, _abi.ptr(tgt), _abi.ptr(src), rows, f.data_ptr(),
                  f.numel(), float(scale), out.data_ptr(), stream())
        ctx.save_for_backward(u, tgt, src, f)
        ctx.scale = float(scale)
        ctx.n_vec = int(unit_vec.shape[0])
        return out

    @staticmethod
    def backward(ctx, gout):
        u, tgt, src, f = ctx.saved_tensors
        grad = fourier_basis_vjp(gout, u, tgt, src, f, ctx.scale)
        return grad, None, None, None, None, None


def fourier_basis_vjp(gout: Tensor, unit_vec: Tensor, target_index: Tensor, source_index: Tensor, freqs: Tensor,
                      scale: float) -> Tensor:
    """grad_unit [E, 3]: the per-row terms (one kernel), then per-vector sums through the CSRs of
    target_index and source_index (fixed order, no atomics)."""
    device = require_cuda(gout, unit_vec)
    u, ld = _unit(unit_vec)
    rows = int(target_index.numel())
    tgt = _index(target_index, rows, "target_index")
    src = _index(source_index, rows, "source_index")
    f = _freqs(freqs, device)
    n_vec = int(u.shape[0])
    grad = torch.zeros((n_vec, 3), dtype=torch.float32, device=device)
    if rows == 0 or n_vec == 0:
        return grad
    g = gout.to(torch.float32).contiguous()
    if g.shape != (rows, 1 + 2 * f.numel()):
        raise ValueError(f"gout must be [{rows}, {1 + 2 * f.numel()}], got {tuple(g.shape)}")
    contrib = torch.empty((rows, 6), dtype=torch.float32, device=device)
    _abi.call("fmd_threebody_fourier_bwd_rows_f32", g.data_ptr(), u.data_ptr(), ld, tgt.data_ptr(), src.data_ptr(),
              rows, f.data_ptr(), f.numel(), float(scale), contrib.data_ptr(), stream())
    segment_sum_csr([(contrib, csr_from_segment(tgt, n_vec), 0, 1.0, None),
                     (contrib, csr_from_segment(src, n_vec), 3, 1.0, None)], n_vec, 3, out=grad)
    return grad


def threebody_fourier_basis(unit_vec: Tensor, target_index: Tensor, source_index: Tensor, freqs: Tensor,
                            scale: float, *, check_range: bool = False) -> Tensor:
    """Reference signature (triton_threebody_fourier.py:273-298); GPU tensors only (the HIP
    kernels have no CPU path). ``check_range`` validates the indices on the host first."""
    return _FourierBasis.apply(unit_vec, target_index, source_index, freqs, float(scale), check_range)


@dataclass(frozen=True)
class LineGraph:
    """The triplet layout of one fixed-capacity line-graph build: per-atom pair offsets and
    short-bond counts, the short-bond matrix [n_atoms, bmax] (directed rows) and the triplet
    rows [t_cap, 5] (atom, pair 1, row 1, pair 2, row 2), whose padding rows the forward reads.
    Every row index is below ``e_cap``, the directed-row capacity of the build."""

    pair_offsets: Tensor  # int64 [n_atoms + 1]
    short_counts: Tensor  # int64 [n_atoms]
    short_edge_matrix: Tensor  # int32 [n_atoms, bmax]
    line_graph: Tensor  # int32 [t_cap, 5]
    e_cap: int
    overflow: Tensor | None = None  # uint8 [1]: the build's overflow flag (all rows padding when set)
    # the segment layouts of the angle -> bond -> atom sums (fmd_nl_line_graph); None when not needed
    short_flags: Tensor | None = None  # uint8 [e_cap]
    short_offsets: Tensor | None = None  # int64 [n_atoms + 1]: CSR of the atoms over bond_rows
    edge_triplet_offsets: Tensor | None = None  # int64 [e_cap + 1]: triplets of each row as first bond
    bond_rows: Tensor | None = None  # int32 [e_cap]: short rows in (atom, rank) order, then -1
    second_perm: Tensor | None = None  # int32 [t_cap]: with edge_triplet_offsets, as second bond

    @property
    def n_atoms(self) -> int:
        return int(self.short_counts.shape[0])

    @property
    def t_cap(self) -> int:
        return int(self.line_graph.shape[0])

    @property
    def bmax(self) -> int:
        return int(self.short_edge_matrix.shape[1])

    @classmethod
    def from_builder(cls, builder) -> "LineGraph":
        if builder.line_graph is None:
            raise ValueError("the builder has no line graph (line_graph_cutoff and t_capacity > 0)")
        return cls(builder.pair_offsets, builder.short_counts, builder.short_edge_matrix, builder.line_graph,
                   builder.e_capacity, builder._overflow, builder.short_flags, builder.short_offsets,
                   builder.edge_triplet_offsets, builder.bond_rows, builder.second_perm)

    def check(self, n_vec: int) -> None:
        if self.pair_offsets.dtype != torch.int64 or self.short_counts.dtype != torch.int64:
            raise ValueError("pair_offsets and short_counts must be int64")
        if self.short_edge_matrix.dtype != torch.int32 or self.line_graph.dtype != torch.int32:
            raise ValueError("short_edge_matrix and line_graph must be int32")
        if self.pair_offsets.shape != (self.n_atoms + 1,) or self.short_edge_matrix.shape[0] != self.n_atoms:
            raise ValueError("pair_offsets / short_edge_matrix do not match short_counts")
        if self.overflow is not None and (self.overflow.dtype != torch.uint8 or self.overflow.numel() != 1):
            raise ValueError("overflow must be one uint8 flag")
        if self.line_graph.dim() != 2 or self.line_graph.shape[1] != 5:
            raise ValueError("line_graph must be [t_cap, 5]")
        for t in (self.pair_offsets, self.short_counts, self.short_edge_matrix, self.line_graph):
            if not t.is_contiguous():
                raise ValueError("line-graph arrays must be contiguous")
        if self.n_atoms <= 0 or self.t_cap <= 0 or self.bmax <= 0:
            raise ValueError("empty line graph")
        if n_vec < self.e_cap:
            raise ValueError(f"unit_vec has {n_vec} rows, the line graph indexes {self.e_cap}")


def _line_args(lg: LineGraph):
    return (lg.pair_offsets.data_ptr(), lg.short_counts.data_ptr(), lg.short_edge_matrix.data_ptr(), lg.bmax)


def _flag(lg: LineGraph):
    return _abi.ptr(lg.overflow)


class _FourierLine(Function):
    @staticmethod
    def forward(ctx, unit_vec, lg, freqs, scale):
        device = require_cuda(unit_vec, lg.line_graph)
        u, ld = _unit(unit_vec)
        lg.check(u.shape[0])
        f = _freqs(freqs, device)
        out = torch.empty((lg.t_cap, 1 + 2 * f.numel()), dtype=torch.float32, device=device)
        _abi.call("fmd_threebody_fourier_line_f32", u.data_ptr(), ld, *_line_args(lg), lg.line_graph.data_ptr(),
                  _flag(lg), lg.n_atoms, lg.t_cap, f.data_ptr(), f.numel(), float(scale), out.data_ptr(), stream())
        ctx.save_for_backward(u, f)
        ctx.lg = lg
        ctx.scale = float(scale)
        return out

    @staticmethod
    def backward(ctx, gout):
        u, f = ctx.saved_tensors
        grad = torch.zeros_like(u)
        fourier_line_vjp(gout, u, ctx.lg, f, ctx.scale, out=grad, accumulate=False)
        return grad, None, None, None


def fourier_line_vjp(gout: Tensor, unit_vec: Tensor, lg: LineGraph, freqs: Tensor, scale: float, *,
                     out: Tensor, accumulate: bool) -> Tensor:
    """Writes (or adds to, with ``accumulate``) the rows of ``out`` [E, >=3] that are short bonds;
    other rows are left as they are (zero them first for a plain gradient)."""
    device = require_cuda(gout, unit_vec, out)
    u, ld = _unit(unit_vec)
    lg.check(u.shape[0])
    f = _freqs(freqs, device)
    g = gout.to(torch.float32).contiguous()
    if g.shape != (lg.t_cap, 1 + 2 * f.numel()):
        raise ValueError(f"gout must be [{lg.t_cap}, {1 + 2 * f.numel()}], got {tuple(g.shape)}")
    o, ldo = rows_view(out)
    if o.data_ptr() != out.data_ptr() or o.shape[0] != u.shape[0] or o.shape[1] < 3 or o.dtype != torch.float32:
        raise ValueError("out must be float32 [E, >= 3] with unit column stride")
    _abi.call("fmd_threebody_fourier_line_bwd_f32", g.data_ptr(), u.data_ptr(), ld, *_line_args(lg), _flag(lg),
              lg.n_atoms, lg.t_cap, f.data_ptr(), f.numel(), float(scale), o.data_ptr(), ldo, 1 if accumulate else 0, stream())
    return out


def threebody_fourier_line(unit_vec: Tensor, line: LineGraph, freqs: Tensor, scale: float) -> Tensor:
    """The basis of every triplet row of a line graph, [t_cap, 1 + 2F]; the VJP is the line
    kernel's (real triplets, deterministic)."""
    return _FourierLine.apply(unit_vec, line, freqs, float(scale))
