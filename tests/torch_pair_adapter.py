"""A pair potential written in plain torch ops behind the adapter protocol, with a padding rule of
the caller's choice (test infrastructure; not collected by pytest).

It reads the published batch the way a third-party model would (the reference's test adapters,
tests/pair_potential_adapter.py:34-133, plug pair potentials in this way): edge vectors from
``edge_index`` / ``edge_image`` / ``cell`` and, under exact-cutoff padding, from
``edge_vec_override`` on the padded rows; per-atom energies over every row of the batch (sink rows
included, the engine sums the first ``n_real``). The potential has an exact cutoff, so a padded
row adds exactly nothing: E_e = 1/2 s_c s_n (1 - (r / rc)^2)^8 for r < rc, else 0.
"""
from __future__ import annotations

import torch
from torch import Tensor, nn

from fastmd_amd.adapters.protocol import CapacityStep, GraphBatch, PaddingRule, TopologySpec


class SmoothPair(nn.Module):
    def __init__(self, cutoff: float = 5.0, power: int = 8, strength: float = 0.08) -> None:
        super().__init__()
        self.cutoff, self.power = float(cutoff), int(power)
        self.strength = nn.Parameter(strength * (1.0 + torch.arange(119, dtype=torch.float32) / 40.0),
                                     requires_grad=False)

    def edge_vectors(self, batch: GraphBatch, positions: Tensor, cell: Tensor) -> Tensor:
        centre = batch.edge_index[:, 0].long()
        neighbour = batch.edge_index[:, 1].long()
        image = batch.edge_image
        shift = image[:, 0:1] * cell[0] + image[:, 1:2] * cell[1] + image[:, 2:3] * cell[2]
        vec = positions.index_select(0, neighbour) + shift - positions.index_select(0, centre)
        if batch.edge_vec_override is not None:
            rows = torch.arange(vec.shape[0], device=vec.device)
            vec = torch.where((rows < batch.n_edges)[:, None], vec, batch.edge_vec_override)
        return vec

    def node_energy(self, batch: GraphBatch, positions: Tensor, cell: Tensor) -> Tensor:
        vec = self.edge_vectors(batch, positions, cell)
        r = torch.linalg.vector_norm(vec, dim=1)
        inside = r < self.cutoff
        base = torch.where(inside, 1.0 - (r / self.cutoff) ** 2, torch.zeros_like(r))
        s = self.strength[batch.species.long()]
        centre = batch.edge_index[:, 0].long()
        pair = s[centre] * s[batch.edge_index[:, 1].long()]
        e = torch.where(inside, 0.5 * pair * base ** self.power, torch.zeros_like(r))
        # per-atom sums in float64 (the grouping of the scatter then does not show in the total)
        return torch.zeros(positions.shape[0], dtype=torch.float64, device=e.device).index_add(0, centre, e.double())


class TorchPairAdapter:
    """``SmoothPair`` as a model adapter with an energy tap (node_energy) and a padding rule."""

    name = "torch_pair"
    compiled = False

    def __init__(self, padding: PaddingRule | None = None, device="cuda", cutoff: float = 5.0) -> None:
        self.module = SmoothPair(cutoff=cutoff).to(device)
        self._padding = padding or PaddingRule("far_self_loops")

    def topology_spec(self) -> TopologySpec:
        return TopologySpec(cutoff=self.module.cutoff, num_interactions=1, model_dtype="float32")

    def padding_rule(self) -> PaddingRule:
        return self._padding

    def capacity_step(self) -> CapacityStep:
        return CapacityStep(u_step=32, min_pad_u=32, u_thermal_factor=1.02)

    def isolated_atom_policy(self) -> str:
        return "model"

    def reference_energies(self):
        return None

    def prepare(self, batch: GraphBatch) -> GraphBatch:
        return batch

    def node_energy(self, inputs: GraphBatch, positions: Tensor, cell: Tensor) -> Tensor:
        return self.module.node_energy(inputs, positions, cell)
