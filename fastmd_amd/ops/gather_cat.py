"""(b) Fused gather + concatenate on the GPU (HIP kernel), with a deterministic VJP.

* ``aligned_gather_cat3(aligned, gathered, index_a, index_b) = cat([aligned, gathered[index_a],
  gathered[index_b]], 1)`` and ``aligned_gather_cat4(aligned, gathered_a, index_a, gathered_b,
  index_b, index_c) = cat([aligned, gathered_a[index_a], gathered_b[index_b],
  gathered_b[index_c]], 1)`` keep the reference's signatures
  (fastmd/models/matris/op/triton_gather_cat.py:181-199, 353-374); widths may differ.
* ``gather_cat(x, src, dst, rbf) = cat([x[src], x[dst], rbf], 1)``: the edge-row form of the
  MD step, ``[E, 2F + R]``.

The VJP sums each gathered block into its source rows with the CSR segment-sum kernel (one
CSR per index; ``src_csr``/``dst_csr`` let the caller pass the neighbour list's own CSRs, the
reverse-edge CSR for senders and the identity CSR for receivers) instead of the reference's
float atomics (triton_gather_cat.py:58-72), so it is deterministic.
"""
from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd._device import require_cuda, rows_view, stream
from fastmd_amd.ops.csr_segment_sum import Csr, csr_from_segment, segment_sum_csr


def _launch(parts, rows: int, out: Tensor) -> None:
    """parts: list of (src matrix, index or None)."""
    srcs, idx, strides, lds, widths, keep = [], [], [], [], [], []
    for src, index in parts:
        if src.dtype != torch.float32:
            raise ValueError(f"gather_cat takes float32 blocks, got {src.dtype}")
        src, ld = rows_view(src)
        stride = 1
        if index is not None:
            if index.dtype != torch.int32 or index.dim() != 1:
                index = index.to(torch.int32).reshape(-1).contiguous()
            stride = index.stride(0) if index.numel() > 1 else 1
            if stride < 1:
                index, stride = index.contiguous(), 1
            if index.numel() != rows:
                raise ValueError(f"index has {index.numel()} entries for {rows} rows")
        elif src.shape[0] != rows:
            raise ValueError(f"aligned block has {src.shape[0]} rows, expected {rows}")
        keep += [src, index]
        srcs.append(src.data_ptr())
        idx.append(None if index is None else index.data_ptr())
        strides.append(stride)
        lds.append(ld)
        widths.append(src.shape[1])
    _abi.call("fmd_gather_cat_f32", len(parts), _abi.ptr_array(srcs), _abi.ptr_array(idx),
              _abi.array(_abi._i64, strides), _abi.array(_abi._i64, lds), _abi.array(_abi._i32, widths), rows, out.data_ptr(), out.stride(0),
              stream())


def _csr_for(index: Tensor, num_rows: int, csr: Csr | None) -> Csr:
    return csr if csr is not None else csr_from_segment(index, num_rows)


class _GatherCat(Function):
    """out = cat(blocks); a block is aligned (row e of its source) or gathered (row index[e])."""

    @staticmethod
    def forward(ctx, kinds, csrs, *tensors):
        # tensors: per block (src, index-or-None)
        blocks = [(tensors[2 * k], tensors[2 * k + 1]) for k in range(len(kinds))]
        rows = None
        for (src, index), kind in zip(blocks, kinds):
            n = index.numel() if kind == "g" else src.shape[0]
            rows = n if rows is None else rows
            if n != rows:
                raise ValueError("gather_cat blocks disagree on the row count")
        width = sum(src.shape[1] for src, _ in blocks)
        require_cuda(*[src for src, _ in blocks])
        out = torch.empty((rows, width), dtype=torch.float32, device=blocks[0][0].device)
        if rows:
            _launch([(src, index if kind == "g" else None) for (src, index), kind in zip(blocks, kinds)], rows, out)
        ctx.kinds = kinds
        ctx.csrs = csrs
        ctx.shapes = [src.shape for src, _ in blocks]
        ctx.save_for_backward(*[index for (_, index) in blocks if index is not None])
        ctx.src_ids = [id(src) for src, _ in blocks]
        return out

    @staticmethod
    def backward(ctx, gout):
        gout = gout.contiguous()
        saved = list(ctx.saved_tensors)
        grads = []
        col = 0
        indices = []
        for kind, shape in zip(ctx.kinds, ctx.shapes):
            indices.append(saved.pop(0) if kind == "g" else None)
        # group gathered blocks by source tensor identity so a shared source sums both blocks
        results: dict[int, Tensor] = {}
        cols = []
        for kind, shape in zip(ctx.kinds, ctx.shapes):
            cols.append(col)
            col += shape[1]
        for k, (kind, shape) in enumerate(zip(ctx.kinds, ctx.shapes)):
            if not ctx.needs_input_grad[2 + 2 * k]:
                grads += [None, None]
                continue
            if kind == "a":
                grads += [gout[:, cols[k]:cols[k] + shape[1]], None]
                continue
            sid = ctx.src_ids[k]
            if sid in results:
                grads += [None, None]  # already summed into the first block of this source
                continue
            terms = []
            for q, (kq, sq) in enumerate(zip(ctx.kinds, ctx.shapes)):
                if kq == "g" and ctx.src_ids[q] == sid:
                    terms.append((gout, _csr_for(indices[q], sq[0], ctx.csrs[q]), cols[q], 1.0, None))
            out = None
            for start in range(0, len(terms), 2):
                out = segment_sum_csr(terms[start:start + 2], shape[0], shape[1], out=out, accumulate=start > 0)
            results[sid] = out
            grads += [out, None]
        return (None, None, *grads)


def _apply(blocks, csrs=None):
    kinds = tuple("a" if index is None else "g" for _, index in blocks)
    csrs = tuple(csrs) if csrs is not None else (None,) * len(blocks)
    flat = []
    for src, index in blocks:
        flat += [src, index]
    return _GatherCat.apply(kinds, csrs, *flat)


def aligned_gather_cat3(aligned: Tensor, gathered: Tensor, index_a: Tensor, index_b: Tensor) -> Tensor:
    """``cat([aligned, gathered[index_a], gathered[index_b]], 1)`` (triton_gather_cat.py:181-199)."""
    return _apply([(aligned, None), (gathered, index_a), (gathered, index_b)])


def aligned_gather_cat4(aligned: Tensor, gathered_a: Tensor, index_a: Tensor, gathered_b: Tensor,
                        index_b: Tensor, index_c: Tensor) -> Tensor:
    """``cat([aligned, gathered_a[index_a], gathered_b[index_b], gathered_b[index_c]], 1)``
    (triton_gather_cat.py:353-374). The VJP of ``gathered_b`` sums both of its blocks in one
    two-term CSR launch (and ``gathered_a`` joins them when it is the same tensor)."""
    return _apply([(aligned, None), (gathered_a, index_a), (gathered_b, index_b), (gathered_b, index_c)])


def gather_cat(x: Tensor, src: Tensor, dst: Tensor, rbf: Tensor, *, src_csr: Csr | None = None,
               dst_csr: Csr | None = None) -> Tensor:
    """Edge rows ``cat([x[src], x[dst], rbf], 1)`` -> ``[E, 2F + R]``. ``src_csr``/``dst_csr``: the
    CSRs of ``src``/``dst`` over the rows of ``x`` for the VJP (built from the indices if None)."""
    return _apply([(x, src), (x, dst), (rbf, None)], csrs=(src_csr, dst_csr, None))
