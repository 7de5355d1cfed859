"""The reference's operator dispatcher (fastmd/engine/dispatch.py:99-556) on this build's HIP ops.

The reference's ``OpDispatcher`` chooses, at each model call site, a Triton kernel or its
PyTorch reference from a ``KernelPolicy`` (switches and row thresholds) and a certified
``ExecutionLayout``. This build has one path: every entry point below runs the HIP kernels (the
deterministic CSR segment sums of ``fastmd_amd.ops.csr_segment_sum`` and the fused gather-cat
of ``fastmd_amd.ops.gather_cat``). There are no switches, no row thresholds and no torch
fallback: CPU tensors raise ``ValueError`` (the HIP kernels have no CPU path), and a missing
native library raises ``NativeLibraryMissing``.

Kept from the reference, with the same names, arguments and meanings:

* ``segment_sum_graph(value, segment, num_segment, graph, side, *, weight=None,
  bin_count=None)`` (:349-369): the CSR segment sum over ``side`` (``"source"`` /
  ``"target"``) of a graph dict, on the side's CSR that ``prepare_segment_csr`` (:303-325) stores
  as ``graph[f"_{side}_segment_sum_csr"] = (perm, offsets, identity, skip_segment)``. The CSR of
  a side is built once from ``graph[f"{side}_index"]`` (a stable sort, so the rows of a segment
  are summed in index order) and cached under the reference's keys
  ``_{side}_segment_attention_perm`` / ``_offsets`` (:604-630). A target side certified sorted
  (``identity_csr``, from the layout) takes the identity CSR from
  ``_target_segment_attention_counts`` or ``_offsets``.
* ``segment_sum(value, segment, num_segment, *, weight=None, bin_count=None)`` (:371-408):
  ``aggregate`` without a weight, ``weighted_segment_sum`` with one (a weight of shape
  ``[rows, D]`` or ``[rows, 1]``).
* ``gather_cat(aligned, gathered, indices)`` (:545-556): ``aligned_gather_cat3`` for one gathered
  tensor, ``aligned_gather_cat4(aligned, gathered[0], indices[0], gathered[1], indices[1],
  indices[2])`` for two.
* ``gather``, ``pair_expand`` and ``pair_average`` (:238-289, :520-522) on the same kernels.
* The predicates ``use_csr_segment_sum``, ``use_weighted_segment_sum``, ``use_gather_cat`` and
  ``use_gather_cat4`` answer whether these kernels take the given tensors (shapes, dtypes and
  device). The HIP gather-cat takes blocks of different widths, so the reference's equal-width
  condition is not one of them.

``dispatcher_for`` (:99-114) caches one dispatcher per (policy, layout, strict_errors,
backend) and refuses a layout that needs communication; ``attach_dispatcher`` (:117-139) stores
the dispatcher under ``"_ops"`` in a processed batch and prepares the CSRs of both graphs.
The reference's other call sites (residual add, segment attention, three-body projections) are
model-specific fusions of MatRIS outside this build's path and are not provided.
"""
from __future__ import annotations

from collections import OrderedDict

import torch
from torch import Tensor

from fastmd_amd._device import require_cuda
from fastmd_amd.ops.csr_segment_sum import csr_from_segment, csr_segment_sum
from fastmd_amd.ops.gather_cat import _apply as _gather_blocks
from fastmd_amd.ops.gather_cat import aligned_gather_cat3, aligned_gather_cat4
from fastmd_amd.ops.segment import aggregate, weighted_segment_sum

_CACHE_SIZE = 256
_DISPATCHERS: OrderedDict[tuple, "OpDispatcher"] = OrderedDict()
_SIDES = ("source", "target")


def _fingerprint(obj) -> object:
    if obj is None:
        return None
    return getattr(obj, "fingerprint", obj)


def _on_gpu(*tensors) -> bool:
    return all(t is None or t.is_cuda for t in tensors)


class OpDispatcher:
    """The single-device operator entry points of the reference's ``OpDispatcher``
    (dispatch.py:142-556) with one HIP path. ``policy`` is kept for the caller (this build has
    no switches); ``layout`` may carry ``route`` (``"identity"`` only) and ``identity_csr`` (the
    graph kinds, ``"atom"`` / ``"line"``, whose target rows are certified sorted)."""

    def __init__(self, policy=None, layout=None, *, strict_errors: bool = False, backend: str | None = None):
        route = getattr(layout, "route", "identity")
        if route != "identity":
            raise ValueError("FastMD supports single-device layouts only")
        self.policy, self.layout = policy, layout
        self.strict_errors, self.backend = bool(strict_errors), backend
        self.key = f"{_fingerprint(policy)}/{_fingerprint(layout)}/{int(self.strict_errors)}/{backend}"
        certified = tuple(getattr(layout, "identity_csr", ()) or ())
        self.identity_csr = {kind: kind in certified for kind in ("atom", "line")}
        # the reference's call sites read this switch before taking segment_sum_graph; the CSR
        # segment sum is the only segment sum here
        self.segment_sum_csr_enabled = True

    def __repr__(self) -> str:
        return (f"OpDispatcher(policy={_fingerprint(self.policy)}, layout={_fingerprint(self.layout)}, "
                f"strict_errors={self.strict_errors}, backend={self.backend})")

    # ------------------------------------------------------------------ pairs

    def pair_expand(self, data: Tensor, directed2undirected: Tensor, graph: dict) -> Tensor:
        """``data[d2u]`` for undirected rows [U, D] -> directed rows [2U, D] (dispatch.py:238-262)."""
        num_undirected = int(graph["num_undirected"])
        if data.dim() != 2 or data.shape[0] != num_undirected:
            raise ValueError(f"pair_expand: data must be [{num_undirected}, D], got {tuple(data.shape)}")
        return self.gather(data, directed2undirected)

    def pair_average(self, data: Tensor, directed2undirected: Tensor, graph: dict) -> Tensor:
        """Mean of the two directed rows of every pair: [2U, D] -> [U, D] (dispatch.py:264-289)."""
        num_undirected = int(graph["num_undirected"])
        if directed2undirected.numel() != 2 * num_undirected:
            raise ValueError(f"pair_average: {directed2undirected.numel()} directed rows for {num_undirected} pairs")
        require_cuda(data, directed2undirected)
        return aggregate(data, directed2undirected, None, average=True, num_segment=num_undirected)

    # ---------------------------------------------------------- segment ops

    def use_weighted_segment_sum(self, weight: Tensor, value: Tensor) -> bool:
        """Whether ``weighted_segment_sum`` takes (weight, value) as they are (dispatch.py:301-306)."""
        return _on_gpu(weight, value) and weight.shape == value.shape and value.dim() == 2

    def use_csr_segment_sum(self, value: Tensor, segment: Tensor, weight: Tensor | None) -> bool:
        """Tensor eligibility of the CSR segment sum (dispatch.py:308-316)."""
        if not (_on_gpu(value, segment, weight) and value.dim() == 2 and value.dtype == torch.float32):
            return False
        if weight is not None and not (weight.shape == value.shape and weight.dtype == value.dtype):
            return False
        return segment.dim() == 1 and segment.numel() == value.shape[0]

    def _side_csr(self, graph: dict, side: str, segment: Tensor, num_segment: int, identity: bool):
        perm_key = f"_{side}_segment_attention_perm"
        off_key = f"_{side}_segment_attention_offsets"
        count_key = f"_{side}_segment_attention_counts"
        if identity:
            off = graph.get(off_key)
            if off is None:
                counts = graph[count_key]
                off = torch.cat((counts.new_zeros(1), counts.cumsum(0))).to(torch.int64)
                graph[off_key] = off
            return None, off, True
        perm, off = graph.get(perm_key), graph.get(off_key)
        if perm is None or off is None:
            require_cuda(segment)
            csr = csr_from_segment(segment, num_segment)
            perm, off = csr.perm, csr.off
            graph[perm_key], graph[off_key] = perm, off
        return perm, off, False

    def prepare_segment_csr(self, graph: dict, num_segment: int) -> None:
        """Store ``(perm, offsets, identity, skip_segment)`` of both sides of ``graph`` as
        ``graph[f"_{side}_segment_sum_csr"]`` (dispatch.py:318-338)."""
        kind = "atom" if graph.get("_topology_graph_kind") == "atom" else "line"
        for side in _SIDES:
            identity = (side == "target" and self.identity_csr[kind]
                        and (f"_{side}_segment_attention_counts" in graph
                             or f"_{side}_segment_attention_offsets" in graph))
            perm, off, identity = self._side_csr(graph, side, graph[f"{side}_index"], int(num_segment), identity)
            graph[f"_{side}_segment_sum_csr"] = (perm, off, identity, -1)

    def segment_csr(self, graph: dict, side: str, segment: Tensor, num_segment: int):
        """The ``(perm, offsets, identity, skip_segment)`` of ``side`` of ``graph``
        (dispatch.py:340-347), prepared on first use."""
        if side not in _SIDES:
            raise ValueError(f"side must be 'source' or 'target', got {side!r}")
        csr = graph.get(f"_{side}_segment_sum_csr")
        if csr is None:
            self.prepare_segment_csr(graph, num_segment)
            csr = graph[f"_{side}_segment_sum_csr"]
        return csr

    def segment_sum_graph(self, value: Tensor, segment: Tensor, num_segment: int, graph: dict, side: str, *,
                          weight: Tensor | None = None, bin_count: Tensor | None = None) -> Tensor:
        """``segment_sum`` over ``side`` of ``graph`` on the side's CSR (dispatch.py:349-369). A
        weight broadcast from ``[rows, 1]`` goes through ``segment_sum``."""
        require_cuda(value, segment, weight)
        if not self.use_csr_segment_sum(value, segment, weight):
            return self.segment_sum(value, segment, num_segment, weight=weight, bin_count=bin_count)
        perm, off, identity, skip_segment = self.segment_csr(graph, side, segment, num_segment)
        return csr_segment_sum(value, segment, num_segment, perm, off, identity, weight=weight,
                               skip_segment=skip_segment)

    def segment_sum(self, value: Tensor, segment: Tensor, num_segment: int, *, weight: Tensor | None = None,
                    bin_count: Tensor | None = None) -> Tensor:
        """``sum_{i in segment s} [weight_i *] value_i`` for ``num_segment`` segments
        (dispatch.py:371-408): ``aggregate`` without a weight, ``weighted_segment_sum`` with one."""
        require_cuda(value, segment, weight)
        if weight is None:
            return aggregate(value, segment, bin_count, average=False, num_segment=num_segment)
        return weighted_segment_sum(weight, value, segment, num_segment)

    # ------------------------------------------------------------ gathers

    def gather(self, value: Tensor, indices: Tensor) -> Tensor:
        """``value[indices]`` (rows) on the gather-cat kernel, with a CSR VJP (dispatch.py:520-522)."""
        require_cuda(value, indices)
        if value.dim() != 2 or indices.dim() != 1:
            raise ValueError(f"gather: value [rows, D] and a 1-D index, got {tuple(value.shape)} and "
                             f"{tuple(indices.shape)}")
        return _gather_blocks([(value, indices)])

    def use_gather_cat(self, aligned: Tensor, gathered: Tensor) -> bool:
        """Whether the 3-part gather-cat takes (aligned, gathered) (dispatch.py:524-530)."""
        return (_on_gpu(aligned, gathered) and aligned.dim() == 2 and gathered.dim() == 2
                and aligned.dtype == gathered.dtype == torch.float32)

    def use_gather_cat4(self, aligned: Tensor, gathered_a: Tensor, gathered_b: Tensor) -> bool:
        """Whether the 4-part gather-cat takes (aligned, gathered_a, gathered_b) (dispatch.py:532-543)."""
        return (self.use_gather_cat(aligned, gathered_a) and gathered_b.is_cuda and gathered_b.dim() == 2
                and gathered_b.dtype == torch.float32)

    def gather_cat(self, aligned: Tensor, gathered, indices) -> Tensor:
        """Fused ``cat([aligned, gathered_k[indices_k]...], 1)`` in 3 or 4 parts (dispatch.py:545-556)."""
        gathered, indices = tuple(gathered), tuple(indices)
        if len(gathered) == 1 and len(indices) == 2:
            return aligned_gather_cat3(aligned, gathered[0], indices[0], indices[1])
        if len(gathered) == 2 and len(indices) == 3:
            return aligned_gather_cat4(aligned, gathered[0], indices[0], gathered[1], indices[1], indices[2])
        raise ValueError(f"gather_cat takes one gathered tensor and two indices, or two and three; got "
                         f"{len(gathered)} and {len(indices)}")


def dispatcher_for(policy=None, layout=None, *, strict_errors: bool = False,
                   backend: str | None = None) -> OpDispatcher:
    """The cached dispatcher of (policy, layout, strict_errors, backend) (dispatch.py:99-114)."""
    key = (_fingerprint(policy), _fingerprint(layout), bool(strict_errors), backend)
    try:
        hash(key)
    except TypeError:
        return OpDispatcher(policy, layout, strict_errors=strict_errors, backend=backend)
    dispatcher = _DISPATCHERS.get(key)
    if dispatcher is not None:
        _DISPATCHERS.move_to_end(key)
        return dispatcher
    dispatcher = OpDispatcher(policy, layout, strict_errors=strict_errors, backend=backend)
    _DISPATCHERS[key] = dispatcher
    if len(_DISPATCHERS) > _CACHE_SIZE:
        _DISPATCHERS.popitem(last=False)
    return dispatcher


def attach_dispatcher(batch_graph: dict, plan=None) -> OpDispatcher:
    """Store the single-device dispatcher under ``"_ops"`` in ``batch_graph`` and in its
    ``atom_graph_dict`` / ``line_graph_dict``, and prepare the CSRs of both graphs
    (dispatch.py:117-139). ``plan``: anything with a ``route`` (``"identity"`` only) and,
    optionally, ``identity_csr``."""
    dispatcher = dispatcher_for(None, plan)
    batch_graph["_ops"] = dispatcher
    atom_graph, line_graph = batch_graph["atom_graph_dict"], batch_graph["line_graph_dict"]
    atom_graph["_ops"] = dispatcher
    line_graph["_ops"] = dispatcher
    dispatcher.prepare_segment_csr(atom_graph, atom_graph["num_segment"])
    if "target_index" in line_graph:
        dispatcher.prepare_segment_csr(line_graph, atom_graph["num_undirected"])
    return dispatcher
