"""(c2) The reference's other segment-sum entry points, on the deterministic CSR kernels.

* ``weighted_segment_sum(weight, value, segment, num_segment)`` =
  ``zeros(num_segment, D).index_add_(0, segment, weight * value)``
  (fastmd/models/matris/op/triton_weighted_segment_sum.py:131-149; its GPU path uses relaxed
  atomics). ``weight`` is [rows, D] or broadcast from [rows, 1].
* ``segment_count(segment, num_segment)`` = ``bincount(segment, minlength=num_segment)`` without a
  host sync (fastmd/engine/kernels/segment.py:42-53).
* ``aggregate(data, segment, bin_count=None, average=True, num_segment=None)``: the segment sum of
  the rows, divided by the (zero-clamped-to-one) counts when ``average`` (segment.py:97-133).

Every sum runs through a CSR of ``segment`` (a stable sort; rows of a segment in index order) and
the fixed-order segment-sum kernel, so results are bitwise reproducible run to run. GPU tensors
only, like the rest of the operator layer.
"""
from __future__ import annotations

import torch
from torch import Tensor

from fastmd_amd._device import require_cuda
from fastmd_amd.ops.csr_segment_sum import csr_from_segment, csr_segment_sum


def _offsets(segment: Tensor, num_segment: int) -> Tensor:
    """CSR offsets [num_segment + 1] of ``segment`` by a sort and a search (no host read)."""
    keys = torch.sort(segment.long())[0]
    bounds = torch.arange(num_segment + 1, device=segment.device, dtype=torch.long)
    return torch.searchsorted(keys, bounds)


def segment_count(segment: Tensor, num_segment: int) -> Tensor:
    """Rows per segment, int64 [num_segment] (segment.py:42-53)."""
    require_cuda(segment)
    if segment.dim() != 1:
        raise ValueError("segment must be 1-D")
    off = _offsets(segment, int(num_segment))
    return off[1:] - off[:-1]


def weighted_segment_sum(weight: Tensor, value: Tensor, segment: Tensor, num_segment: int) -> Tensor:
    """``sum over rows r with segment[r] == s of weight[r] * value[r]`` (triton_weighted_segment_sum.py:131-149),
    differentiable in ``weight`` and ``value``."""
    require_cuda(weight, value, segment)
    if value.dim() != 2:
        raise ValueError("value must be 2-D")
    if weight.shape != value.shape:
        if weight.dim() != 2 or weight.shape[0] != value.shape[0] or weight.shape[1] != 1:
            raise ValueError(f"weight must be {tuple(value.shape)} or ({value.shape[0]}, 1), got {tuple(weight.shape)}")
        weight = weight.expand_as(value).contiguous()
    num_segment = int(num_segment)
    csr = csr_from_segment(segment, num_segment)
    return csr_segment_sum(value, segment, num_segment, perm=csr.perm, off=csr.off, weight=weight)


def aggregate(data: Tensor, segment: Tensor, bin_count: Tensor | None = None, average: bool = True,
              num_segment: int | None = None) -> Tensor:
    """Sum (``average``: mean) of the rows of ``data`` per segment (segment.py:97-133). Without
    ``num_segment`` the segment count is read from the device (one host sync, as the reference's
    ``bincount`` path)."""
    require_cuda(data, segment, bin_count)
    if num_segment is None:
        num_segment = int(segment.max().item()) + 1 if segment.numel() else 0
        if bin_count is not None:
            num_segment = max(num_segment, int(bin_count.shape[0]))
    num_segment = int(num_segment)
    csr = csr_from_segment(segment, num_segment)
    out = csr_segment_sum(data, segment, num_segment, perm=csr.perm, off=csr.off)
    if not average:
        return out
    if bin_count is None:
        bin_count = csr.off[1:] - csr.off[:-1]
    if bin_count.shape[0] != num_segment:
        bin_count = torch.cat([bin_count, bin_count.new_ones(num_segment - bin_count.shape[0])])
    bin_count = bin_count.where(bin_count != 0, bin_count.new_ones(1))
    return (out.T / bin_count).T
