"""(c) Deterministic CSR segment sums on the GPU (HIP kernels, no float atomics).

``csr_segment_sum`` keeps the signature and semantics of the reference's
``fastmd/models/matris/op/triton_csr_segment_sum.py:433-479``:

    out[s] = sum_{segment[i] == s} [weight[i] *] value[i]

over a CSR (``off`` int64 [num_segment + 1], ``perm`` int32/int64 [rows], or the identity
when rows are sorted by segment), with ``skip_segment`` giving a zero row and zero gradient.
Its VJP is the transpose kernel (gvalue[r] = gout[seg r] (* weight[r]), gweight[r] =
gout[seg r] * value[r]), deterministic as well. Rows past ``off[num_segment]`` of an identity
CSR belong to no segment (the padding rows of a fixed-capacity edge list): they add nothing
and get zero gradient.

``Csr`` carries a CSR; ``segment_sum_csr`` is the multi-term primitive the model kernels use
(sum of up to two CSR terms, each with its own rows, permutation and sign).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd._device import require_cuda, rows_view, stream


@dataclass(frozen=True)
class Csr:
    """A CSR over rows: run of segment s is ``[off[s], off[s+1])`` clamped to ``rows`` rows of
    the value matrix; row j of a run is ``perm[j]`` (None: the identity)."""

    off: Tensor  # int64 [num_segment + 1] on the device
    perm: Tensor | None = None  # int32 [>= off[-1]] on the device, entries < 0 skipped
    rows: int | None = None  # clamp of the runs (None: the value's row count)

    @property
    def num_segment(self) -> int:
        return int(self.off.shape[0]) - 1


def csr_from_segment(segment: Tensor, num_segment: int) -> Csr:
    """The CSR of an arbitrary segment index (stable order within a segment). Host plumbing:
    torch's stable sort and a count; the hot path gets its CSRs from the neighbour list."""
    segment = segment.long()
    perm = torch.argsort(segment, stable=True).to(torch.int32)
    counts = torch.bincount(segment, minlength=num_segment)[:num_segment]
    off = torch.zeros(num_segment + 1, dtype=torch.int64, device=segment.device)
    torch.cumsum(counts, 0, out=off[1:])
    return Csr(off, perm)


def _prep_off(off: Tensor) -> Tensor:
    if off.dtype != torch.int64 or not off.is_contiguous():
        off = off.to(torch.int64).contiguous()
    return off


def _prep_perm(perm: Tensor | None) -> Tensor | None:
    if perm is None:
        return None
    if perm.dtype != torch.int32 or not perm.is_contiguous():
        perm = perm.to(torch.int32).contiguous()
    return perm


def segment_sum_csr(terms, num_segment: int, dim: int, *, out: Tensor | None = None, accumulate: bool = False,
                    skip_segment: int = -1) -> Tensor:
    """``out[s] = sum_t scale_t * sum_{j in run_t(s)} [w_t[r] *] v_t[r, col_t:col_t+dim]``.

    ``terms``: up to two tuples ``(value [rows, >= col+dim] fp32, csr: Csr, col: int, scale: float,
    weight: Tensor | None)``. No autograd (the model's backward kernels call it directly)."""
    if not 1 <= len(terms) <= 2:
        raise ValueError("segment_sum_csr takes one or two terms")
    first = terms[0][0]
    device = require_cuda(*[t[0] for t in terms])
    if out is None:
        out = (torch.zeros if accumulate else torch.empty)((num_segment, dim), dtype=torch.float32, device=device)
    values, lds, cols, weights, scales, perms, offs, rows = [], [], [], [], [], [], [], []
    keep = []
    for value, csr, col, scale, weight in terms:
        if value.dtype != torch.float32:
            raise ValueError(f"segment sums take float32 values, got {value.dtype}")
        value, ld = rows_view(value)
        if col < 0 or col + dim > value.shape[1]:
            raise ValueError("column block out of range")
        if csr.num_segment != num_segment:
            raise ValueError(f"CSR has {csr.num_segment} segments, expected {num_segment}")
        off = _prep_off(csr.off)
        perm = _prep_perm(csr.perm)
        if weight is not None:
            weight, wld = rows_view(weight)
            if wld != ld or weight.shape != value.shape:
                raise ValueError("weight must have the value's shape and layout")
        n_rows = value.shape[0] if csr.rows is None else min(int(csr.rows), value.shape[0])
        if perm is not None and n_rows > 0 and perm.numel() == 0:
            raise ValueError("empty permutation")
        keep += [value, off, perm, weight]
        values.append(value.data_ptr())
        lds.append(ld)
        cols.append(col)
        weights.append(None if weight is None else weight.data_ptr())
        scales.append(float(scale))
        perms.append(None if perm is None else perm.data_ptr())
        offs.append(off.data_ptr())
        rows.append(n_rows if perm is None else min(n_rows, perm.numel()))
    out2, ldo = rows_view(out)
    if out2.data_ptr() != out.data_ptr():
        raise ValueError("out must have unit column stride")
    _abi.call("fmd_segsum_csr_f32", len(terms), _abi.ptr_array(values), _abi.array(_abi._i64, lds),
              _abi.array(_abi._i64, cols),
              None if all(w is None for w in weights) else _abi.ptr_array(weights),
              _abi.array(_abi._f32, scales),
              None if all(p is None for p in perms) else _abi.ptr_array(perms),
              _abi.ptr_array(offs), _abi.array(_abi._i64, rows), num_segment, dim, skip_segment,
              1 if accumulate else 0, out.data_ptr(), ldo, stream())
    del keep, first
    return out


def segment_sum_t(gout: Tensor, csr: Csr, n_rows: int, *, value: Tensor | None = None, weight: Tensor | None = None,
                  need_value_grad: bool = True, need_weight_grad: bool = False, skip_segment: int = -1):
    """Transpose of one CSR term (see module docstring): ``(gvalue, gweight)``."""
    require_cuda(gout)
    gout, ldg = rows_view(gout.contiguous() if gout.dtype == torch.float32 else gout.float().contiguous())
    dim = gout.shape[1]
    off = _prep_off(csr.off)
    perm = _prep_perm(csr.perm)
    rows = n_rows if csr.rows is None else min(n_rows, int(csr.rows))
    gv = torch.empty((n_rows, dim), dtype=torch.float32, device=gout.device) if need_value_grad else None
    gw = torch.empty((n_rows, dim), dtype=torch.float32, device=gout.device) if need_weight_grad else None
    if gv is None and gw is None:
        return None, None
    vld = 0
    if value is not None:
        value, vld = rows_view(value)
    if weight is not None:
        weight, wld = rows_view(weight)
        if value is not None and wld != vld:
            raise ValueError("weight and value must share a layout")
        vld = wld if value is None else vld
    if rows < n_rows and perm is None:
        # runs clamped below the row count: rows past the clamp are zeroed by the kernel via off
        pass
    _abi.call("fmd_segsum_csr_t_f32", gout.data_ptr(), ldg, _abi.ptr(value), _abi.ptr(weight), vld,
              _abi.ptr(perm), off.data_ptr(), csr.num_segment, rows, dim, skip_segment, _abi.ptr(gv),
              _abi.ptr(gw), stream())
    if rows < n_rows:
        if gv is not None:
            gv[rows:].zero_()
        if gw is not None:
            gw[rows:].zero_()
    return gv, gw


class _CsrSegmentSum(Function):
    @staticmethod
    def forward(ctx, value, weight, num_segment, csr_off, csr_perm, skip_segment):
        csr = Csr(csr_off, csr_perm)
        out = segment_sum_csr([(value, csr, 0, 1.0, weight)], num_segment, value.shape[1],
                              skip_segment=skip_segment)
        ctx.save_for_backward(value, weight, csr_off, csr_perm)
        ctx.skip_segment = skip_segment
        return out

    @staticmethod
    def backward(ctx, gout):
        value, weight, off, perm = ctx.saved_tensors
        need_v = ctx.needs_input_grad[0]
        need_w = ctx.needs_input_grad[1] and weight is not None
        gv, gw = segment_sum_t(gout, Csr(off, perm), value.shape[0], value=value if need_w else None,
                               weight=weight if need_v else None, need_value_grad=need_v,
                               need_weight_grad=need_w, skip_segment=ctx.skip_segment)
        return gv, gw, None, None, None, None


def csr_segment_sum(value: Tensor, segment: Tensor | None, num_segment: int, perm: Tensor | None = None,
                    off: Tensor | None = None, identity_perm: bool = False, *, weight: Tensor | None = None,
                    skip_segment: int = -1) -> Tensor:
    """Reference signature (triton_csr_segment_sum.py:433-479). GPU tensors only: the HIP
    kernels have no CPU path (use ``torch.index_add_`` on the CPU)."""
    if value.dim() != 2:
        raise ValueError(f"value must be 2D, got shape {tuple(value.shape)}")
    if weight is not None and (weight.shape != value.shape or weight.dtype != value.dtype):
        raise ValueError(f"weight must match value, got {tuple(weight.shape)}/{weight.dtype} and "
                         f"{tuple(value.shape)}/{value.dtype}")
    num_segment = int(num_segment)
    skip_segment = int(skip_segment)
    if skip_segment < -1 or skip_segment >= num_segment:
        raise ValueError("skip_segment must be -1 or an existing private segment")
    if segment is not None and (segment.dim() != 1 or segment.numel() != value.shape[0]):
        raise ValueError(f"segment must have one entry per row ({value.shape[0]}), got {tuple(segment.shape)}")
    if identity_perm and off is None:
        raise ValueError("identity CSR metadata requires offsets")
    require_cuda(value, weight, segment, perm, off)
    if value.dtype != torch.float32:
        raise ValueError("csr_segment_sum: float32 values only")
    if identity_perm:
        perm = None
    elif perm is None or off is None:
        if segment is None:
            raise ValueError("a segment index or a CSR is required")
        csr = csr_from_segment(segment, num_segment)
        perm, off = csr.perm, csr.off
    return _CsrSegmentSum.apply(value, weight, num_segment, _prep_off(off), _prep_perm(perm), skip_segment)
