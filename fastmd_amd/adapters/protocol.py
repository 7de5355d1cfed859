"""The model plugin boundary of the GPU-resident MD step.

Same types, field names and meanings as the reference's ``fastmd/adapters/protocol.py``
(TopologySpec :48-65, PaddingRule :68-119, GraphBatch :144-211, ModelAdapter :214-253,
EnergyTap :276-295, CapacityStep :324-374, CaptureContract :401-437), restricted to what the
edges-only single-system path reads. A model plugs in by exposing these; the Morse pair
potential and the MACE-like model of this package do.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Literal, Protocol, runtime_checkable

from torch import Tensor, nn


@dataclass(frozen=True)
class TopologySpec:
    """The graph a model consumes (protocol.py:48-65)."""

    cutoff: float
    num_interactions: int
    triplet_cutoff: float | None = None
    undirected_pairs: bool = False
    model_dtype: Literal["float32", "float64"] = "float32"
    edge_order: Literal["sorted", "by_centre"] = "sorted"
    max_neighbors: int | None = None


@dataclass(frozen=True)
class PaddingRule:
    """What the padded rows of a fixed-capacity edge list look like (protocol.py:68-119).

    ``far_self_loops``: padded row k is a self-loop of real atom ``k mod n_real`` with an integer
    image along the longest lattice vector, at least ``min_length`` and twice the cutoff long
    (with a line graph a padded triplet joins a padded pair to itself at that pair's atom).
    ``exact_rc_loops``: padded row k is a self-loop of real atom ``k mod n_real`` with image 0,
    whose edge vector the model takes from ``GraphBatch.edge_vec_override`` (``pad_vector``,
    by default (cutoff, 0, 0)); edges only. ``sink_atoms``: the batch has ``n_dummy`` sink rows
    after the real ones (at the origin, atomic number 1); padded row k is a self-loop of a sink
    with image (3, 3, 3), both rows of a padded pair on one sink, the padded pairs (and
    triplets) spread evenly over the sinks; the model leaves the sink rows out (``n_real``).
    """

    kind: Literal["sink_atoms", "far_self_loops", "exact_rc_loops"] = "far_self_loops"
    min_length: float = 0.0
    pad_vector: tuple[float, float, float] | None = None
    placement: Literal["round_robin"] = "round_robin"

    def __post_init__(self) -> None:
        if self.kind not in ("sink_atoms", "far_self_loops", "exact_rc_loops"):
            raise ValueError(f"PaddingRule: unknown kind {self.kind!r}")
        if self.placement != "round_robin":
            raise ValueError(f"PaddingRule: unknown placement {self.placement!r}")
        if not math.isfinite(self.min_length) or self.min_length < 0.0:
            raise ValueError("PaddingRule: min_length must be finite and >= 0")
        if self.min_length and self.kind != "far_self_loops":
            raise ValueError("PaddingRule: min_length applies to far_self_loops only")
        if self.pad_vector is not None:
            if self.kind != "exact_rc_loops":
                raise ValueError("PaddingRule: pad_vector applies to exact_rc_loops only")
            if len(self.pad_vector) != 3 or not all(math.isfinite(v) for v in self.pad_vector):
                raise ValueError("PaddingRule: pad_vector must be three finite numbers")


@dataclass
class SystemSegments:
    """Several systems in one batch (protocol.py:123-141; the field names are the reference's).
    System s owns the rows [row_ptr[s], row_ptr[s + 1]) (its slot); its atoms are the first
    ``atoms[s]`` of them (None: all), the rest are vacant rows with no candidate and no real edge.
    No edge joins two systems. ``cells`` [count, 3, 3] float32 holds each system's cell (None: the
    batch's one cell). All are persistent device buffers."""

    count: int
    row_ptr: Tensor  # [count + 1] int64
    system_of_row: Tensor  # [rows] int32
    cells: Tensor | None = None
    atoms: Tensor | None = None


def require_atom_rows(batch, model: str) -> None:
    """Raise unless every row of ``batch`` is a model row: this package's HIP models read the
    padded rows of far self-loop or exact-cutoff padding (which they skip by the edge count) but
    not the extra rows of sink padding."""
    if batch.positions is not None and batch.positions.shape[0] != batch.n_real:
        raise ValueError(f"the {model} model takes far_self_loops or exact_rc_loops padding, not sink rows "
                         f"({batch.positions.shape[0] - batch.n_real} rows past n_real)")


def system_rows(batch) -> int | None:
    """Device address of the batch's per-row system index (None for one system): the argument
    the edge-geometry kernel takes to form each edge's image in its own system's cell."""
    systems = getattr(batch, "systems", None)
    return None if systems is None or systems.cells is None else systems.system_of_row.data_ptr()


@dataclass
class GraphBatch:
    """The graph a builder publishes: engine-owned persistent buffers (protocol.py:144-211).

    Edges are directed, listed in both directions; real rows ``[0, n_edges)`` sorted by (centre,
    neighbour, image), then padding rows laid out by ``padding``. Edge vector of row e:
    ``positions[edge_index[e, 1]] + edge_image[e] @ cell - positions[edge_index[e, 0]]``.

    Beyond the reference's fields, a fixed-capacity batch of this package carries its CSR by
    centre (``edge_offsets``, int64 [n_real + 1], real rows only) and the reverse row of every
    real edge (``edge_reverse``, int32 [rows], -1 on padding), from which the deterministic
    segment sums over receivers and senders are formed without atomics.
    """

    positions: Tensor | None
    frac_coords: Tensor
    cell: Tensor
    species: Tensor
    n_real: int
    edge_index: Tensor
    edge_image: Tensor
    n_edges: Tensor | None
    cutoff: float
    padding: PaddingRule | None
    edge_vec_override: Tensor | None = None
    triplet_cutoff: float | None = None
    pair_d2u: Tensor | None = None
    pair_u2d: Tensor | None = None
    triplets: Tensor | None = None
    status: Any = None
    composition: str = ""
    evidence: Any = None
    systems: Any = None
    edge_offsets: Tensor | None = None
    edge_reverse: Tensor | None = None
    line: Any = None  # the line graph's arrays (fastmd_amd.ops.threebody.LineGraph) when built
    # a permutation of the atom rows in a spatial (Morton) order, refreshed with the candidates:
    # kernels that take one atom per wave visit them in this order (same results, L2 locality)
    atom_order: Tensor | None = None
    # rows of the largest system in the batch (replica or slot union; 0: all rows one system):
    # kernels whose arithmetic is chosen by system size choose it by this
    max_system_rows: int = 0
    # slot unions: (first row, rows, atoms) of every slot, host ints; kernels whose arithmetic is
    # chosen by system size choose it per slot from its atoms (empty: one system or equal replicas)
    system_slots: tuple = ()

    @property
    def edge_dst(self) -> Tensor:
        """The centre (receiving) atom of each edge."""
        return self.edge_index[:, 0]

    @property
    def edge_src(self) -> Tensor:
        """The neighbour (sending) atom of each edge."""
        return self.edge_index[:, 1]


@dataclass(frozen=True)
class CapacityStep:
    """A model's capacity tiers (protocol.py:324-374): pair step, minimum pad, thermal factor."""

    u_step: int = 512
    min_pad_u: int = 256
    u_thermal_factor: float = 1.0
    t_step: int | None = None
    min_pad_t: int | None = None
    t_thermal_factor: float = 1.0


@dataclass(frozen=True)
class CaptureContract:
    """What a model promises about one call (protocol.py:401-437)."""

    sync_free: bool = True
    exact_cutoff: bool = True
    accuracy_class: str = "fp32_noise"
    force_mode: str = "engine_autograd"
    stress_unit: str = "eV/A^3"
    compiled: str = "none"


@runtime_checkable
class ModelAdapter(Protocol):
    """A model behind the runtime (protocol.py:214-253)."""

    name: str
    module: nn.Module
    compiled: bool

    def topology_spec(self) -> TopologySpec: ...

    def padding_rule(self) -> PaddingRule: ...

    def prepare(self, batch: GraphBatch) -> Any: ...

    def isolated_atom_policy(self) -> Literal["reference", "error", "model"]: ...

    def reference_energies(self) -> Tensor | None: ...


@runtime_checkable
class EnergyTap(Protocol):
    """Capability: per-atom energies that the engine differentiates itself (protocol.py:276-295)."""

    def node_energy(self, inputs: Any, positions: Tensor, cell: Tensor) -> Tensor: ...
