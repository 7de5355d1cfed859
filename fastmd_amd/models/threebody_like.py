"""A CHGNet/MatRIS-style three-body interatomic potential whose forward and VJP run as HIP kernels.

The reference's three-body models are upstream CHGNet (wrapped by fastmd/models/chgnet.py:1-60,
356-366) and MatRIS (fastmd/models/matris/model.py, interaction_block.py); neither's weights nor
the upstream chgnet package are available here, so this package defines its own configs[4] model
"64 channels, 4 layers, atom graph 6 A, bond graph 3 A, angles expanded in Fourier terms" with
the reference's data path: the line graph of the fixed-capacity builder (bonds = directed edges
shorter than the bond cutoff, triplets = ordered pairs of distinct bonds at a centre), the
Fourier angle basis (triton_threebody_fourier.py), the triplet gather and the segment sums
angles -> bonds -> atoms.

Model (per layer t; atom features h [N, C], bond features eps [E, C] on every directed edge):
  edge e = (centre i <- neighbour j): vec, r, u = vec / r, ef_n = sqrt(2/rc) sin(n pi r/rc)/r fc(r)
  (n = 1..8), fc the polynomial cutoff 1 - 21x^5 + 35x^6 - 15x^7 at rc = 6 A; bond envelope
  s(r) = the same polynomial at rb (bonds: r < rb), 0 on other rows.
  triplet k = (i; bond b1, bond b2): alpha_k = [1/sqrt2, sin(theta f), cos(theta f)] / sqrt(pi),
  theta = acos((u_b1 . u_b2)(1 - 1e-6)), f = 1..F
  h = embedding[Z]; eps = ef We
  three-body:  z3_k = eps_b1 W3a + eps_b2 W3b + h_i W3c + alpha_k W3d        ([T, C])
               eps_b += (1 / avg_angles) sum_{k: b1 = b} silu(z3_k) s_b1 s_b2    (angles -> bonds)
  atom update: z2_e = h_j W2a + h_i W2b + eps_e W2c                           ([E, C])
               h_i += (1 / avg_neighbors) sum_{e: centre i} silu(z2_e) fc_e         (edges -> atoms)
  readout:     E_i = e0[Z_i] + h_i . wr
Random init from ``torch.Generator().manual_seed(seed)``.

dE/dpos is formed by explicit VJP kernels (one autograd node). Atom update: the gated-sum VJP
gives the pre-activation gradients gz2, their per-centre sums and the cutoff gradient; by
linearity the node gradient is the product of the per-centre and per-sender sums with the weight
blocks, so only gz2 W2c^T is formed on the edge rows. Three-body update: per triplet gz3 and the
envelope terms, ga3 = gz3 W3^T on the triplet rows (far fewer than the edges), then per bond the
sums over its triplets as first and as second bond, per atom over its triplets. The Fourier VJP
runs once over all layers' angle gradients.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
from torch import Tensor, nn
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd.adapters.protocol import (CapacityStep, CaptureContract, GraphBatch, PaddingRule, TopologySpec,
                                         require_atom_rows, system_rows)
from fastmd_amd.ops.csr_segment_sum import Csr, segment_sum_csr
from fastmd_amd.ops.threebody import LineGraph, fourier_line_vjp
from fastmd_amd.ops.wide_gemm import gemm, gemm_gather, gemm_group, split_planes

_ELEMENTS = 118
# pairs and triplets in tiers of 128 with at least 128 of padding, held at 1.01x the pair and 1.06x
# the triplet demand (the CHGNet adapter's tiers, fastmd/models/chgnet.py:25-30)
_CAPACITY_STEP = CapacityStep(u_step=128, min_pad_u=128, u_thermal_factor=1.01, t_step=128, min_pad_t=128,
                              t_thermal_factor=1.06)


@dataclass(frozen=True)
class ThreeBodyConfig:
    channels: int = 64
    num_interactions: int = 4
    n_basis: int = 8
    cutoff: float = 6.0
    bond_cutoff: float = 3.0
    n_freq: int = 4  # 1 + 2 * 4 = 9 angle columns: the constant and 8 Fourier terms
    avg_num_neighbors: float = 15.0
    avg_num_angles: float = 4.0
    elements: tuple = (55, 50, 53)
    seed: int = 0


class ThreeBodyLike(nn.Module):
    """Parameters (frozen, float32), matrices stored [in, out]."""

    def __init__(self, config: ThreeBodyConfig = ThreeBodyConfig()) -> None:
        super().__init__()
        self.config = config
        C, nb, A = config.channels, config.n_basis, 1 + 2 * config.n_freq
        if C % 64 or not 64 <= C <= 256:
            raise ValueError("channels must be 64, 128, 192 or 256")
        if not 0.0 < config.bond_cutoff <= config.cutoff:
            raise ValueError("the bond cutoff must lie in (0, cutoff]")
        nel = len(config.elements)
        gen = torch.Generator().manual_seed(config.seed)

        def rnd(*shape, fan_in=None):
            std = 1.0 / math.sqrt(fan_in) if fan_in else 1.0
            return nn.Parameter(torch.randn(*shape, generator=gen) * std, requires_grad=False)

        self.embedding = rnd(nel, C)
        self.We = rnd(nb, C, fan_in=nb)
        self.layers = nn.ModuleList()
        for _ in range(config.num_interactions):
            layer = nn.Module()
            layer.W3 = rnd(3 * C + A, C, fan_in=3 * C + A)  # [eps_b1; eps_b2; h_i; alpha]
            layer.W2 = rnd(3 * C, C, fan_in=3 * C)  # [h_j; h_i; eps_e]
            self.layers.append(layer)
        self.wr = rnd(C, fan_in=C)
        self.e0 = nn.Parameter(-1.0 - torch.rand(nel, generator=gen), requires_grad=False)
        self.register_buffer("freqs", torch.arange(1, config.n_freq + 1, dtype=torch.float32))
        table = torch.full((_ELEMENTS + 1,), -1, dtype=torch.int32)
        for k, z in enumerate(config.elements):
            table[z] = k
        self.register_buffer("z_table", table)

    @property
    def fourier_scale(self) -> float:
        return math.sqrt(math.pi)

    def _cached(self, key, build):
        """Derived weight layouts, rebuilt when a parameter changes in place (version counter)."""
        params = [p for p in self.parameters()]
        stamp = tuple((p.data_ptr(), p._version) for p in params)
        cache = self.__dict__.setdefault("_layout_cache", {})
        hit = cache.get(key)
        if hit is None or hit[0] != stamp:
            hit = (stamp, build())
            cache[key] = hit
        return hit[1]

    def layouts(self) -> dict:
        C = self.config.channels

        def build():
            out = {"w3t": [], "w2_je_t": [], "w2_i": [], "w3_vjp": [], "w2_nodes": [], "w2_eps": []}
            for layer in self.layers:
                W3, W2 = layer.W3.detach(), layer.W2.detach()
                out["w3t"].append(W3[:3 * C].t().contiguous())  # [C, 3C] (N, K): the triplet GEMM
                # the edge GEMM on [h_j | eps_e] ([C, 2C] (N, K)); the centre block h_i W2b per atom
                out["w2_je_t"].append(torch.cat([W2[:C], W2[2 * C:]], 0).t().contiguous())
                out["w2_i"].append(W2[C:2 * C].contiguous())  # [C, C] ([K, N])
                out["w3_vjp"].append(W3[:3 * C].contiguous())  # [3C, C] (N, K): gz3 [W3a; W3b; W3c]^T
                out["w2_nodes"].append(torch.cat([W2[:C], W2[C:2 * C]], 1).contiguous())  # [C, 2C] VJP
                out["w2_eps"].append(W2[2 * C:].contiguous())  # [C, C] VJP
            out["w3d"] = torch.cat([layer.W3.detach()[3 * C:] for layer in self.layers], 1).contiguous()  # [A, L C]
            # the VJP group's weights as bf16 planes (its split-plane form; K = 2C and C)
            out["w2_nodes_planes"] = [split_planes(w) for w in out["w2_nodes"]]
            out["w2_eps_planes"] = [split_planes(w) for w in out["w2_eps"]]
            return out

        return self._cached("layouts", build)


@dataclass
class ThreeBodyInput:
    batch: GraphBatch
    line: LineGraph
    elem: Tensor  # int32 [rows]
    csr_dst: Csr = field(default=None)
    csr_src: Csr = field(default=None)


def _call(name, *args):
    _abi.call(name, *args, _abi.stream_handle())


def _empty(*shape, device, dtype=torch.float32):
    return torch.empty(*shape, dtype=dtype, device=device)


class _Saved:
    """What the forward keeps for the VJP (the autograd ctx, or this holder outside autograd)."""


def _forward(ctx, positions: Tensor, cell: Tensor, model: ThreeBodyLike, inputs: ThreeBodyInput) -> Tensor:
    cfg = model.config
    batch, lg = inputs.batch, inputs.line
    dev = positions.device
    C, nb, L = cfg.channels, cfg.n_basis, cfg.num_interactions
    A = 1 + 2 * cfg.n_freq
    n = positions.shape[0]
    e_cap, t_cap = batch.edge_index.shape[0], lg.t_cap
    if positions.dtype != torch.float32:
        raise ValueError("the three-body model runs in float32")
    if lg.e_cap != e_cap or lg.edge_triplet_offsets is None:
        raise ValueError("the line graph does not match the edge list")
    positions = positions.detach().contiguous()
    cell = cell.detach().to(torch.float32).contiguous()
    ei, off, n_edges = batch.edge_index, batch.edge_offsets, batch.n_edges
    lay = model.layouts()
    geo = _empty(e_cap, 8, device=dev)
    ef = _empty(e_cap, nb, device=dev)
    de = _empty(e_cap, nb, device=dev)
    _call("fmd_edge_geometry_f32", positions.data_ptr(), cell.data_ptr(), system_rows(batch), ei.data_ptr(),
          batch.edge_image.data_ptr(),
          n_edges.data_ptr(), e_cap, float(cfg.cutoff), nb, geo.data_ptr(), ef.data_ptr(), de.data_ptr())
    _call("fmd_tb_bond_envelope_f32", geo.data_ptr(), lg.short_flags.data_ptr(), n_edges.data_ptr(), e_cap,
          float(cfg.bond_cutoff))
    # the angle basis of every triplet row and its products with all layers' angle blocks
    alpha = _empty(t_cap, A, device=dev)
    _call("fmd_threebody_fourier_line_f32", geo.data_ptr(), 8, lg.pair_offsets.data_ptr(), lg.short_counts.data_ptr(),
          lg.short_edge_matrix.data_ptr(), lg.bmax, lg.line_graph.data_ptr(), _abi.ptr(lg.overflow), lg.n_atoms,
          t_cap, model.freqs.data_ptr(), cfg.n_freq, model.fourier_scale, alpha.data_ptr())
    aw = gemm(alpha, lay["w3d"], b_layout=1)  # [T, L C]
    h = _empty(n, C, device=dev)
    _call("fmd_embed_f32", inputs.elem.data_ptr(), model.embedding.data_ptr(), n, C, h.data_ptr())
    eps = gemm(ef, model.We, b_layout=1)  # [E, C]
    line = lg.line_graph
    row1, row2, atom = line[:, 2], line[:, 4], line[:, 0]
    inv_ang, inv_avg = 1.0 / cfg.avg_num_angles, 1.0 / cfg.avg_num_neighbors
    saved = []
    for t in range(L):
        # three-body update of the bonds: gather-cat [eps_b1 | eps_b2 | h_i] fused into the GEMM's
        # load, the angle block added per row
        z3 = gemm_gather([(eps, row1), (eps, row2), (h, atom)], lay["w3t"][t], row_add=(aw[:, t * C:(t + 1) * C], None))
        _call("fmd_tb_bond_sum_f32", z3.data_ptr(), C, C, geo.data_ptr(), lg.short_offsets.data_ptr(),
              lg.bond_rows.data_ptr(), lg.edge_triplet_offsets.data_ptr(), lg.line_graph.data_ptr(), lg.n_atoms,
              t_cap, inv_ang, eps.data_ptr(), C)
        # atom update: [h_j | eps_e] gathered into the GEMM's load, the centre block h_i W2b formed
        # once per atom and added per row
        q2 = gemm(h, lay["w2_i"][t], b_layout=1)
        z2 = gemm_gather([(h, ei[:, 1]), (eps, None)], lay["w2_je_t"][t], row_add=(q2, ei[:, 0]))
        _call("fmd_tb_gated_sum_f32", z2.data_ptr(), C, e_cap, C, geo[:, 4:].data_ptr(), 8, None, None, 0,
              off.data_ptr(), n, inv_avg, h.data_ptr(), C, 1)
        saved.append((z3, z2))
    energy = _empty(n, device=dev)
    _call("fmd_tb_readout_f32", h.data_ptr(), C, C, model.wr.data_ptr(), inputs.elem.data_ptr(), model.e0.data_ptr(),
          n, energy.data_ptr())
    ctx.model, ctx.inputs, ctx.saved = model, inputs, saved
    ctx.geo, ctx.de = geo, de
    ctx.n, ctx.e_cap = n, e_cap
    return energy


def _vjp(ctx, gE: Tensor | None, sign: float, stress_cell: Tensor | None = None):
    """sign * dE/dpos [n, 3] (gE None: the gradient of the plain sum of the node energies); with
    ``stress_cell`` (the unstrained float32 cell) also the stress [3, 3]: ``(forces, stress)``."""
    model, inputs = ctx.model, ctx.inputs
    cfg = model.config
    lg, batch = inputs.line, inputs.batch
    C, nb, L = cfg.channels, cfg.n_basis, cfg.num_interactions
    n, e_cap, t_cap = ctx.n, ctx.e_cap, lg.t_cap
    dev = ctx.geo.device
    geo = ctx.geo
    lay = model.layouts()
    inv_ang, inv_avg = 1.0 / cfg.avg_num_angles, 1.0 / cfg.avg_num_neighbors
    off = batch.edge_offsets

    gh = _empty(n, C, device=dev)
    _call("fmd_tb_readout_bwd_f32", _abi.ptr(gE), 1.0, model.wr.data_ptr(), C, n, gh.data_ptr(), C)
    # stored by the first layer the loop takes (the last), added to by the others: no zero fills
    geps = _empty(e_cap, C, device=dev)
    gfc = _empty(e_cap, device=dev)
    gs = _empty(e_cap, device=dev)  # written on the bond rows only (read there only)
    gz3_all = _empty(t_cap, L * C, device=dev)
    gz2 = _empty(e_cap, C, device=dev)
    s_dst = _empty(n, C, device=dev)
    gsw = _empty(t_cap, 2, device=dev)
    per_atom = Csr(lg.pair_offsets, None, t_cap)
    for t in reversed(range(L)):
        z3, z2 = ctx.saved[t]
        first = t == L - 1
        # atom update: gz2 and its per-centre sums; the cutoff's gradient accumulates over layers
        _call("fmd_tb_gated_sum_bwd_f32", gh.data_ptr(), C, z2.data_ptr(), C, e_cap, C, geo[:, 4:].data_ptr(), 8, None,
              None, 0, off.data_ptr(), n, inv_avg, gz2.data_ptr(), C, s_dst.data_ptr(), C, gfc.data_ptr(), 1,
              0 if first else 1)
        s_src = segment_sum_csr([(gz2, inputs.csr_src, 0, 1.0, None)], n, C)
        # gh += [S_src | S_dst] [W2a; W2b]^T and geps += gz2 W2c^T in one launch
        # (the split-plane form of the group, weights split once: 0.91 -> 0.86 ms/step at 5 000
        # atoms against the fp32 MFMA tiles)
        gemm_group([{"a": s_src, "a2": s_dst, "b": lay["w2_nodes"][t], "b_planes": lay["w2_nodes_planes"][t],
                     "out": gh, "accumulate": True},
                    {"a": gz2, "b": lay["w2_eps"][t], "b_planes": lay["w2_eps_planes"][t], "out": geps,
                     "accumulate": not first}], b_layout=0)
        # three-body update: gz3 per triplet (this layer's column block) and its envelope terms,
        # ga3 = gz3 [W3a; W3b; W3c]^T on the triplet rows, then per bond the sums of its triplets as
        # first and second bond into geps (and gs), per atom those of its triplets into gh
        gz3 = gz3_all[:, t * C:(t + 1) * C]
        _call("fmd_tb_triplet_bwd_f32", geps.data_ptr(), C, z3.data_ptr(), C, C, geo.data_ptr(),
              lg.line_graph.data_ptr(), lg.pair_offsets.data_ptr(), n, t_cap, inv_ang, gz3.data_ptr(), L * C,
              gsw.data_ptr())
        ga3 = gemm(gz3, lay["w3_vjp"][t], b_layout=0)  # [T, 3C]
        _call("fmd_tb_bond_reduce_f32", ga3.data_ptr(), 3 * C, C, gsw.data_ptr(), lg.short_offsets.data_ptr(),
              lg.bond_rows.data_ptr(), lg.edge_triplet_offsets.data_ptr(), lg.second_perm.data_ptr(), n, t_cap,
              geps.data_ptr(), C, gs.data_ptr(), 0 if first else 1)
        segment_sum_csr([(ga3, per_atom, 2 * C, 1.0, None)], n, C, out=gh, accumulate=True)
    # the angle basis: all layers' angle gradients at once, then the Fourier VJP (short rows)
    galpha = gemm(gz3_all, lay["w3d"], b_layout=0)  # [T, A]
    gu = _empty(e_cap, 3, device=dev)  # written on the bond rows only (read there only)
    fourier_line_vjp(galpha, geo[:, :3], lg, model.freqs, model.fourier_scale, out=gu, accumulate=False)
    gef = gemm(geps, model.We, b_layout=0)  # [E, nb]
    gvec = _empty(e_cap, 3, device=dev)
    _call("fmd_tb_geometry_bwd_f32", geo.data_ptr(), ctx.de.data_ptr(), nb, gef.data_ptr(), nb, gu.data_ptr(), 3,
          gfc.data_ptr(), gs.data_ptr(), lg.short_flags.data_ptr(), batch.n_edges.data_ptr(), e_cap, gvec.data_ptr())
    forces = segment_sum_csr([(gvec, inputs.csr_src, 0, sign, None), (gvec, inputs.csr_dst, 0, -sign, None)], n, 3)
    if stress_cell is None:
        return forces
    from fastmd_amd.engine.energy_derivative import edge_stress

    # the angles enter through the bond unit vectors, whose gradient is part of gvec: the virial
    # of the edge vectors is the whole strain derivative
    return forces, edge_stress(geo, gvec, batch.n_edges, stress_cell)


class _ThreeBodyEnergy(Function):
    """positions -> node energies [rows]; backward: dE/dpos by the VJP kernels."""

    @staticmethod
    def forward(ctx, positions, cell, model: ThreeBodyLike, inputs: ThreeBodyInput):
        return _forward(ctx, positions, cell, model, inputs)

    @staticmethod
    def backward(ctx, gE):
        gE = gE.detach().to(torch.float32).contiguous()
        return _vjp(ctx, gE, 1.0), None, None, None


class ThreeBodyAdapter:
    """The three-body model as a ModelAdapter with an EnergyTap (chgnet.py's surface: line-graph
    topology, far self-loop padding, pair and triplet capacity tiers)."""

    name = "threebody_like"
    compiled = False

    def __init__(self, module: ThreeBodyLike | None = None, *, config: ThreeBodyConfig | None = None,
                 device: torch.device | str = "cuda") -> None:
        module = module if module is not None else ThreeBodyLike(config or ThreeBodyConfig())
        self.module = module.to(device).eval()
        for p in self.module.parameters():
            p.requires_grad_(False)

    def topology_spec(self) -> TopologySpec:
        cfg = self.module.config
        return TopologySpec(cutoff=float(cfg.cutoff), num_interactions=int(cfg.num_interactions),
                            triplet_cutoff=float(cfg.bond_cutoff), undirected_pairs=True, model_dtype="float32",
                            edge_order="sorted")

    def padding_rule(self) -> PaddingRule:
        return PaddingRule("far_self_loops")

    def capacity_step(self) -> CapacityStep:
        return _CAPACITY_STEP

    def capture_contract(self) -> CaptureContract:
        return CaptureContract(sync_free=True, exact_cutoff=True, accuracy_class="fp32_noise",
                               force_mode="engine_autograd", stress_unit="eV/A^3", compiled="none")

    def isolated_atom_policy(self) -> str:
        return "model"

    def reference_energies(self) -> Tensor:
        row = torch.full((1, _ELEMENTS), float("nan"), dtype=torch.float64)
        for k, z in enumerate(self.module.config.elements):
            row[0, z - 1] = float(self.module.e0[k])
        return row

    def prepare(self, batch: GraphBatch) -> ThreeBodyInput:
        """Aliases of the batch and its line graph, the element index of every row (host check of
        the species, outside any graph) and the two CSRs of the edge list."""
        if batch.positions is None or batch.edge_offsets is None or batch.edge_reverse is None:
            raise ValueError("the three-body model needs a fixed-capacity batch with its CSR")
        require_atom_rows(batch, "three-body")
        if batch.line is None or batch.line.edge_triplet_offsets is None:
            raise ValueError("the three-body model reads a line graph (a builder with line_graph_cutoff)")
        if abs(float(batch.triplet_cutoff) - float(self.module.config.bond_cutoff)) > 1e-12:
            raise ValueError(f"line graph cutoff {batch.triplet_cutoff} != the model's bond cutoff "
                             f"{self.module.config.bond_cutoff}")
        species = batch.species.long()
        table = self.module.z_table.to(species.device)
        if bool(((species < 1) | (species > _ELEMENTS)).any()) or bool((table[species.clamp(1, _ELEMENTS)] < 0).any()):
            raise ValueError(f"the three-body model supports atomic numbers {list(self.module.config.elements)}")
        elem = table[species].to(torch.int32).contiguous()
        rows = batch.edge_index.shape[0]
        return ThreeBodyInput(batch=batch, line=batch.line, elem=elem, csr_dst=Csr(batch.edge_offsets, None, rows),
                              csr_src=Csr(batch.edge_offsets, batch.edge_reverse, rows))

    def node_energy(self, inputs: ThreeBodyInput, positions: Tensor, cell: Tensor) -> Tensor:
        if cell.requires_grad:
            raise NotImplementedError("stress (a strained cell) is not supported by the three-body kernels")
        return _ThreeBodyEnergy.apply(positions, cell, self.module, inputs)

    def energy_and_forces(self, inputs: ThreeBodyInput, positions: Tensor, cell: Tensor,
                          segments=1) -> tuple[Tensor, Tensor]:
        """(E [1] float64, F = -dE/dpos [rows, 3]) by the forward and VJP kernels, without autograd."""
        from fastmd_amd.engine.energy_derivative import sum_f64_segments

        saved = _Saved()
        energies = _forward(saved, positions.detach(), cell.detach(), self.module, inputs)
        energy = sum_f64_segments(energies, segments)  # one energy per replica or system
        return energy, _vjp(saved, None, -1.0)

    def energy_forces_stress(self, inputs: ThreeBodyInput, positions: Tensor, cell: Tensor):
        """``energy_and_forces`` plus the stress dE/d(strain) / V [3, 3] float32 of one system
        (energy_derivative.py:110-140)."""
        from fastmd_amd.engine.energy_derivative import sum_f64_into

        saved = _Saved()
        energies = _forward(saved, positions.detach(), cell.detach(), self.module, inputs)
        energy = sum_f64_into(energies)
        forces, stress = _vjp(saved, None, -1.0, stress_cell=cell.detach().to(torch.float32).contiguous())
        return energy, forces, stress
