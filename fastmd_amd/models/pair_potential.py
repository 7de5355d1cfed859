"""Morse pair potential of the plumbing configuration, on the HIP kernels.

D = 0.3 eV, a = 1.5 / Angstrom, r0 = 3.0 Angstrom, cutoff 6 Angstrom, shifted to zero at
the cutoff: V(r) = D [(1 - exp(-a (r - r0)))^2 - 1] - V(rc) for r < rc, E_i = 1/2 sum_j V(r_ij).
The reference's tests plug pair potentials in through the same adapter protocol
(tests/pair_potential_adapter.py:34-265, ``SmoothPairPotential`` with an exact cutoff); this is
one such adapter, with an EnergyTap the engine differentiates.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import Tensor, nn
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd.adapters.protocol import (CapacityStep, GraphBatch, PaddingRule, TopologySpec, require_atom_rows,
                                         system_rows)
from fastmd_amd.ops.csr_segment_sum import Csr, segment_sum_csr


class Morse(nn.Module):
    def __init__(self, D: float = 0.3, a: float = 1.5, r0: float = 3.0, cutoff: float = 6.0) -> None:
        super().__init__()
        self.D, self.a, self.r0, self.cutoff = float(D), float(a), float(r0), float(cutoff)
        self.vshift = self.D * ((1 - math.exp(-self.a * (self.cutoff - self.r0))) ** 2 - 1)


@dataclass
class PairInput:
    batch: GraphBatch
    csr_dst: Csr
    csr_src: Csr


class _MorseEnergy(Function):
    @staticmethod
    def forward(ctx, positions, cell, model: Morse, inputs: PairInput):
        batch = inputs.batch
        dev = positions.device
        n = positions.shape[0]
        e_cap = batch.edge_index.shape[0]
        positions = positions.detach().contiguous()
        cell = cell.detach().to(torch.float32).contiguous()
        geo = torch.empty(e_cap, 8, dtype=torch.float32, device=dev)
        ef = torch.empty(e_cap, 1, dtype=torch.float32, device=dev)
        de = torch.empty(e_cap, 1, dtype=torch.float32, device=dev)
        s = _abi.stream_handle()
        _abi.call("fmd_edge_geometry_f32", positions.data_ptr(), cell.data_ptr(), system_rows(batch),
                  batch.edge_index.data_ptr(),
                  batch.edge_image.data_ptr(), batch.n_edges.data_ptr(), e_cap, model.cutoff, 1, geo.data_ptr(),
                  ef.data_ptr(), de.data_ptr(), s)
        energy = torch.empty(n, dtype=torch.float32, device=dev)
        dvdr = torch.empty(e_cap, dtype=torch.float32, device=dev)
        _abi.call("fmd_morse_f32", geo.data_ptr(), batch.edge_offsets.data_ptr(), batch.n_edges.data_ptr(), e_cap, n,
                  model.D, model.a, model.r0, model.cutoff, model.vshift, energy.data_ptr(), dvdr.data_ptr(), s)
        ctx.geo, ctx.dvdr, ctx.inputs, ctx.n, ctx.e_cap = geo, dvdr, inputs, n, e_cap
        return energy

    @staticmethod
    def backward(ctx, gE):
        gE = gE.detach().to(torch.float32).contiguous()
        return _morse_vjp(ctx, gE, 1.0)[0], None, None, None


class _Saved:
    """What the forward keeps for the VJP outside autograd."""


def _morse_vjp(ctx, gE: Tensor, sign: float, stress_cell: Tensor | None = None):
    """(sign * dE/dpos [rows, 3] with E = sum_i gE_i E_i, and with ``stress_cell`` the stress
    [3, 3] of the edge-vector gradient, else None)."""
    batch = ctx.inputs.batch
    gvec = torch.empty(ctx.e_cap, 3, dtype=torch.float32, device=gE.device)
    _abi.call("fmd_morse_bwd_f32", ctx.geo.data_ptr(), ctx.dvdr.data_ptr(), batch.edge_index.data_ptr(),
              gE.data_ptr(), batch.n_edges.data_ptr(), ctx.e_cap, gvec.data_ptr(), _abi.stream_handle())
    gpos = segment_sum_csr([(gvec, ctx.inputs.csr_src, 0, sign, None), (gvec, ctx.inputs.csr_dst, 0, -sign, None)],
                           ctx.n, 3)
    if stress_cell is None:
        return gpos, None
    from fastmd_amd.engine.energy_derivative import edge_stress

    return gpos, edge_stress(ctx.geo, gvec, batch.n_edges, stress_cell)


class MorsePairAdapter:
    name = "morse"
    compiled = False

    def __init__(self, module: Morse | None = None, device="cuda") -> None:
        self.module = (module or Morse()).to(device)

    def topology_spec(self) -> TopologySpec:
        return TopologySpec(cutoff=self.module.cutoff, num_interactions=1, model_dtype="float32")

    def padding_rule(self) -> PaddingRule:
        return PaddingRule("far_self_loops")

    def capacity_step(self) -> CapacityStep:
        return CapacityStep(u_step=32, min_pad_u=32, u_thermal_factor=1.02)

    def isolated_atom_policy(self) -> str:
        return "model"

    def reference_energies(self):
        return None

    def prepare(self, batch: GraphBatch) -> PairInput:
        if batch.edge_offsets is None or batch.edge_reverse is None:
            raise ValueError("the pair potential needs an edges-only batch with its CSR")
        require_atom_rows(batch, "Morse")
        rows = batch.edge_index.shape[0]
        return PairInput(batch, Csr(batch.edge_offsets, None, rows), Csr(batch.edge_offsets, batch.edge_reverse, rows))

    def node_energy(self, inputs: PairInput, positions: Tensor, cell: Tensor) -> Tensor:
        if cell.requires_grad:
            raise NotImplementedError("a strained cell is not differentiated by the pair-potential kernels: "
                                      "stress comes from energy_forces_stress")
        return _MorseEnergy.apply(positions, cell, self.module, inputs)

    def energy_forces_stress(self, inputs: PairInput, positions: Tensor, cell: Tensor):
        """(E [1] float64, F = -dE/dpos [rows, 3], stress dE/d(strain) / V [3, 3] float32) of one
        system (energy_derivative.py:110-140): the forward and VJP kernels of ``node_energy`` with
        a unit energy seed, and the virial of the VJP's edge-vector gradient."""
        from fastmd_amd.engine.energy_derivative import sum_f64_into

        saved = _Saved()
        energies = _MorseEnergy.forward(saved, positions.detach(), cell.detach(), self.module, inputs)
        seed = torch.ones_like(energies)
        forces, stress = _morse_vjp(saved, seed, -1.0, stress_cell=cell.detach().to(torch.float32).contiguous())
        return sum_f64_into(energies), forces, stress
