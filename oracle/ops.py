"""Operator oracle (test infrastructure only; see oracle/__init__.py).

The reference's CPU branches of the three fused ops, in float64 NumPy:
  gather-cat: ``torch.cat([aligned, gathered[a], gathered[b]], 1)`` (triton_gather_cat.py:192-199)
  segment sum: ``zeros(num_segment, D).index_add_(0, segment, rows)`` (triton_csr_segment_sum.py:463-479)
  GEMM: ``F.linear`` (triton_wide_gemm.py:488-489)
plus the algebraic VJPs (scatter-add of the gathered blocks, gather of the segment rows).
"""
from __future__ import annotations

import numpy as np


def gather_cat(blocks):
    """blocks: list of (matrix, index or None) -> concatenated rows (exact copy)."""
    cols = [m if idx is None else m[np.asarray(idx)] for m, idx in blocks]
    return np.concatenate(cols, axis=1)


def segment_sum(value, segment, num_segment, weight=None):
    rows = np.asarray(value, dtype=np.float64)
    if weight is not None:
        rows = rows * np.asarray(weight, dtype=np.float64)
    out = np.zeros((num_segment, rows.shape[1]))
    np.add.at(out, np.asarray(segment), rows)
    return out


def segment_sum_vjp(gout, segment, weight=None, value=None):
    g = np.asarray(gout, dtype=np.float64)[np.asarray(segment)]
    gv = g if weight is None else g * weight
    gw = None if value is None else g * value
    return gv, gw


def linear(x, w, b=None):
    y = np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T
    return y if b is None else y + b


def relative(a, b) -> float:
    """max |a - b| / max |b| (the reference's relative(), tests/adapters/test_mace_adapter.py:270-273)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    scale = np.max(np.abs(b)) if b.size else 0.0
    return float(np.max(np.abs(a - b)) / scale) if scale > 0 else float(np.max(np.abs(a - b), initial=0.0))
