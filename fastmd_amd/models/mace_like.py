"""A MACE-like equivariant interatomic potential whose forward and backward run as HIP kernels.

The reference's MACE family is third-party (mace-torch 0.3.16, wrapped by
fastmd/models/mace.py:254-477); it is not available here, so this build defines its own
"2-layer, 128-channel, L_max = 1, correlation-order-3, 8-Bessel" model with the same plugin
surface (``MACEAdapter``-shaped adapter: far self-loop padding, CapacityStep(32, 32, 1.02),
an EnergyTap the engine differentiates) and puts the configs' operators on its path:
the gather-cat (b), the wide edge GEMM (d) and the receiver segment sums (c).

Model (per interaction layer t, node features h0 [N, C] scalars and h1 [N, 3, C] vectors):
  edge e = (centre i <- neighbour j), vec = pos_j + image @ cell - pos_i, r = |vec|, u = vec / r
  ef_n   = sqrt(2/rc) sin(n pi r / rc) / r * fcut(r),  n = 1..8;  fcut = 1 - 21x^5 + 35x^6 - 15x^7
  a_e    = [h0_j | h0_i | ef_e]                                 (gather-cat, [E, 2C + 8])
  z_e    = a_e @ W1                                              ([2C+8, 4C]) evaluated as
         = P_j + Q_i + ef_e @ W1[2C:],  P = h0 W1[:C], Q = h0 W1[C:2C]  (node-factored, the default:
           node GEMMs, the radial term added per row in the message kernels), or as the edge GEMM
           over the gather-cat rows (fused into its operand load; FACTORED_Z off)
  w_e    = silu(z_e) * fcut(r)  = (wa | wb | wc | wd)             (h1 = 0: wa | wb only)
  m0     = wa h0_j + wc (h1_j . u),  m1_x = wb h0_j u_x + wd h1_j,x
  A0_i, A1_i = (1 / avg_num_neighbors) * sum over the rows of i   (segment sums)
  P0 = A0 Wm0, P1_x = A1_x Wm1;  n1 = |P1|^2
  B0 = c1 P0 + c2 P0^2 + c3 n1 + c4 P0^3 + c5 P0 n1          (element-dependent c, d)
  B1_x = (d1 + d2 P0 + d3 P0^2 + d4 n1) P1_x
  h0' = B0 Wo0 + h0 Wsc0,  h1'_x = B1_x Wo1                    (last layer: scalars only)
readout: E_i = E0[Z_i] + scale * (h0^(1) . wr1 + silu(h0^(2) Wr2a) . wr2b) + shift.
Initial h0 = embedding[Z], h1 = 0. Random init from ``torch.manual_seed(seed)``.

The gradient dE/dpos is formed by explicit VJP kernels (fmd_mace_*_bwd), not by autograd of
many small ops: the whole model is ONE autograd node whose backward launches ~25 kernels.
Padding rows (far self-loops beyond the cutoff) contribute exactly zero and are skipped.
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
from fastmd_amd.ops.wide_gemm import (Planes, gemm, gemm_gather, gemm_group, gemm_planes, gemm_splitk,
                                     split_planes)

_ELEMENTS = 118
_CAPACITY_STEP = CapacityStep(u_step=32, min_pad_u=32, u_thermal_factor=1.02)
# edge lists from this many rows form the receiver block of the edge GEMM per atom (below it the
# two extra node GEMMs cost more launch latency than the halved edge GEMM saves)
HOIST_MIN_ROWS = 16384
# the node side of each layer (two GEMMs, the contraction, three GEMMs; and its VJP) as one fused
# launch per direction (fmd_mace_node_fwd/bwd_f32) instead of the chain of six. Off: each 32-atom
# tile walks its phases' 24 K-slices one after the other, which measured slower (50 us per launch
# at 135 atoms, 73 / 117 us at 10 000) than the six short launches it replaces; kept tested
# against the oracle beside the chain.
FUSED_NODE = False
# Node-factored edge pre-activation: z_e = [h0_j | h0_i | ef_e] W1 is linear in its blocks, so the
# layer forms P = h0 W1[:C] and Q = h0 W1[C:2C] per atom (node GEMMs; the first layer's, of the
# element embedding, as per-element tables) and the message kernels add the radial term
# ef_e W1[2C:] per row: no [E, 4C] edge array is written or read and no edge GEMM runs. Off: z
# is the edge GEMM over the gather-cat rows (the configs' wide-GEMM operator on the path), kept
# tested against the oracle beside the factored form.
FACTORED_Z = True
# The energy launch forms the float64 total itself (its last workgroup) up to this many atoms; above,
# a separate one-workgroup sum: each of the energy launch's workgroups fences at device scope, which
# took that launch from 7 to 60 us at 10 000 atoms (2 500 workgroups).
ENERGY_TOTAL_MAX_ATOMS = 2048
# The first layer's output GEMM adds the per-element residual and next-layer rows in its epilogue
# (above the small-system sizes) instead of accumulating onto outputs prefilled with them.
ROWS_IN_EPILOGUE = True
# Merged node side (node-factored, unfused, two or more layers): a layer's output GEMM launch
# also forms the next layer's P and Q, the last one the readout's first product (its h0n is
# never formed), and the first layer's per-element rows come from one gather launch. Off: one
# launch per product, as the unmerged chain (kept tested against the oracle).
MERGED_NODE = True
# Systems of at most this many atoms (each system of a slot union by its own count) split each
# atom's rows over four waves in the message kernels (one wave per atom leaves a small system's
# chip idle while each wave walks its rows); the per-atom sums are then added over the waves.
SPLIT_ROWS_MAX_ATOMS = 2048
# Launches of at most this many atoms (unfused node side) form P0, P1 and the contraction in one
# launch (fmd_mace_mix_symcon_f32: 16 atoms x 16 channels per workgroup, the scalar and vector
# rows of a tile in its four waves), and in the VJP gB0, gB1 and the contraction's VJP in one
# (fmd_mace_mix_symcon_bwd_f32), the residual's input gradient then joining the gA group. Above,
# the grouped GEMMs and the contraction kernels run as separate launches.
SMALL_NODE_MAX_ATOMS = 2048


@dataclass(frozen=True)
class MaceLikeConfig:
    channels: int = 128
    num_interactions: int = 2
    n_basis: int = 8
    cutoff: float = 6.0
    avg_num_neighbors: float = 15.0
    readout_hidden: int = 16
    elements: tuple = (55, 50, 53)
    scale: float = 1.0
    shift: float = 0.0
    seed: int = 0


class MaceLike(nn.Module):
    """Parameters of the model (frozen, float32). Node-side matrices are stored [in, out]; the
    edge GEMM weight W1 is [2C + 8, 4C]."""

    def __init__(self, config: MaceLikeConfig = MaceLikeConfig()) -> None:
        super().__init__()
        self.config = config
        C, nb, H = config.channels, config.n_basis, config.readout_hidden
        if C % 64 or C // 64 not in (1, 2, 4):
            raise ValueError("channels must be 64, 128 or 256")
        nel = len(config.elements)
        gen = torch.Generator().manual_seed(config.seed)

        def rnd(*shape, fan_in=None):
            std = 1.0 / math.sqrt(fan_in) if fan_in else 1.0
            return nn.Parameter(torch.randn(*shape, generator=gen) * std, requires_grad=False)

        self.embedding = rnd(nel, C)
        self.layers = nn.ModuleList()
        for t in range(config.num_interactions):
            layer = nn.Module()
            layer.W1 = rnd(2 * C + nb, 4 * C, fan_in=2 * C + nb)
            layer.Wm0 = rnd(C, C, fan_in=C)
            layer.Wm1 = rnd(C, C, fan_in=C)
            layer.Wc = rnd(nel, 5, C, fan_in=5)
            layer.Wd = rnd(nel, 4, C, fan_in=4)
            layer.Wo0 = rnd(C, C, fan_in=C)
            layer.Wo1 = rnd(C, C, fan_in=C)
            layer.Wsc0 = rnd(C, C, fan_in=C)
            self.layers.append(layer)
        self.wr1 = rnd(C, fan_in=C)
        self.Wr2a = rnd(C, H, fan_in=C)
        self.wr2b = rnd(H, fan_in=H)
        self.e0 = nn.Parameter(-1.0 - torch.rand(nel, generator=gen), requires_grad=False)
        table = torch.full((_ELEMENTS + 1,), -1, dtype=torch.int32)
        for k, z in enumerate(config.elements):
            table[z] = k
        self.register_buffer("z_table", table)

    @property
    def r_max(self) -> float:
        return self.config.cutoff

    def w1_t(self, t: int) -> Tensor:
        """W1 of layer t stored K-contiguous ([4C, 2C + 8]) for the edge GEMM, which is fastest with
        both operands K-contiguous; rebuilt when W1 is changed in place (version counter)."""
        w = self.layers[t].W1
        key = (w.data_ptr(), w._version, w.device)
        cache = self.__dict__.setdefault("_w1t_cache", {})
        hit = cache.get(t)
        if hit is None or hit[0] != key:
            hit = (key, w.detach().t().contiguous())
            cache[t] = hit
        return hit[1]

    def node_weights(self, t: int) -> dict:
        """Layer t's node-side weights in the layouts of the fused node kernels ([columns, K],
        K-contiguous): wm0t = Wm0^T, wm1t = Wm1^T, wout0 = [Wo0; Wsc0]^T, wout1 = [Wo1; 0]^T (forward)
        and wo0st = [Wo0; Wsc0], wo1st = [Wo1; 0] (VJP), and wo1t = Wo1^T for the grouped forward
        GEMMs; "planes" holds the bf16 planes of the grouped GEMMs' [N, K] weights (forward: wm0t,
        wm1t, wout0, wo1t; VJP: Wo0, Wo1, Wsc0, Wm0, Wm1); rebuilt when a weight changes in place."""
        layer = self.layers[t]
        mats = (layer.Wm0, layer.Wm1, layer.Wo0, layer.Wo1, layer.Wsc0)
        key = tuple((w.data_ptr(), w._version, w.device) for w in mats)
        cache = self.__dict__.setdefault("_node_w_cache", {})
        hit = cache.get(t)
        if hit is None or hit[0] != key:
            wm0, wm1, wo0, wo1, wsc0 = (w.detach() for w in mats)
            zero = torch.zeros_like(wo1)
            w = {"wm0t": wm0.t().contiguous(), "wm1t": wm1.t().contiguous(),
                 "wout0": torch.cat([wo0, wsc0], 0).t().contiguous(),
                 "wout1": torch.cat([wo1, zero], 0).t().contiguous(),
                 "wo0st": torch.cat([wo0, wsc0], 0).contiguous(),
                 "wo1st": torch.cat([wo1, zero], 0).contiguous(), "wo1t": wo1.t().contiguous(),
                 "wo0t": wo0.t().contiguous()}
            src = {"wm0t": w["wm0t"], "wm1t": w["wm1t"], "wout0": w["wout0"], "wo1t": w["wo1t"], "Wo0": wo0,
                   "Wo1": wo1, "Wsc0": wsc0, "Wm0": wm0, "Wm1": wm1, "wo0t": w["wo0t"]}
            w["planes"] = {name: split_planes(x.contiguous()) for name, x in src.items()}
            hit = (key, w)
            cache[t] = hit
        return hit[1]

    def skip_table(self) -> Tensor:
        """The first layer's residual term per element, embedding @ Wsc0 ([elements, C]), formed in
        float64 and rounded once to float32; rebuilt when either weight changes in place. The
        first layer's input is the embedding, so h0 @ Wsc0 is the same row for every atom of an
        element and its float32 rounding error is the same for all of them: accumulated inside
        the output GEMM that error grows with |B0 Wo0|, so it adds to the energy coherently over
        the atoms and with a size that follows the configuration (an energy error the forces do
        not share, seen as drift of the NHC conserved quantity)."""
        mats = (self.embedding, self.layers[0].Wsc0)
        key = tuple((w.data_ptr(), w._version, w.device) for w in mats)
        hit = self.__dict__.get("_skip_cache")
        if hit is None or hit[0] != key:
            table = (self.embedding.detach().double() @ self.layers[0].Wsc0.detach().double()).float().contiguous()
            hit = (key, table)
            self.__dict__["_skip_cache"] = hit
        return hit[1]

    def w1_receiver_t(self, t: int) -> Tensor:
        """The receiver rows of W1 ([C, 2C)) stored K-contiguous ([4C, C])."""
        w = self.layers[t].W1
        C = self.config.channels
        key = (w.data_ptr(), w._version, w.device)
        cache = self.__dict__.setdefault("_w1r_cache", {})
        hit = cache.get(t)
        if hit is None or hit[0] != key:
            hit = (key, w.detach()[C:2 * C].t().contiguous())
            cache[t] = hit
        return hit[1]

    def w1_sender_t(self, t: int) -> Tensor:
        """The sender and radial rows of W1 ([0, C) and [2C, 2C + nb)) stored K-contiguous
        ([4C, C + nb]): the edge GEMM's weight once the receiver block is formed per atom."""
        w = self.layers[t].W1
        C = self.config.channels
        key = (w.data_ptr(), w._version, w.device)
        cache = self.__dict__.setdefault("_w1s_cache", {})
        hit = cache.get(t)
        if hit is None or hit[0] != key:
            hit = (key, torch.cat([w.detach()[:C], w.detach()[2 * C:]], 0).t().contiguous())
            cache[t] = hit
        return hit[1]

    def w1_sender_node_t(self, t: int) -> Tensor:
        """The sender rows of W1 ([0, C)) stored K-contiguous ([4C, C]): the B operand of the
        node-factored P = h0 W1[:C]."""
        w = self.layers[t].W1
        C = self.config.channels
        key = (w.data_ptr(), w._version, w.device)
        cache = self.__dict__.setdefault("_w1sn_cache", {})
        hit = cache.get(t)
        if hit is None or hit[0] != key:
            hit = (key, w.detach()[:C].t().contiguous())
            cache[t] = hit
        return hit[1]

    def merged_weights(self) -> dict:
        """Products of consecutive weights for the merged node side (float64, rounded once, with
        the bf16 planes of the GEMM operands; rebuilt when any weight changes in place):
          "pq_next"[t] (t < L - 1): the next layer's P and Q straight from this layer's
            [B0 | h0] (h0n = B0 Wo0 + h0 Wsc0, so h0n W1' = B0 (Wo0 W1') + h0 (Wsc0 W1')), as
            [N, K] operands: (Wo0 W1'[:, :4C])^T ([4C, C]) in the first layer, whose residual
            enters as a per-element table, and ([Wo0; Wsc0] W1'[:, :4C])^T ([4C, 2C]) later;
          "y": the readout's first product from the last layer's [B0 | h0], ([Wo0; Wsc0] Wr2a)^T
            ([H, 2C]), so the last h0n is never formed;
          "gy": (Wo0 Wr2a, Wsc0 Wr2a) of the last layer ([C, H] each): its VJP's first products
            straight from dE/dy;
          "tables": the first layer's per-element rows: the residual embedding Wsc0 ([nel, C]) and
            its next-layer blocks (embedding Wsc0) W1'[:C / C:2C, :4C] ([nel, 4C] each)."""
        mats = [self.embedding, self.Wr2a] + [w for layer in self.layers for w in (layer.W1, layer.Wo0, layer.Wsc0)]
        key = tuple((w.data_ptr(), w._version, w.device) for w in mats)
        hit = self.__dict__.get("_merged_cache")
        if hit is None or hit[0] != key:
            C, L = self.config.channels, len(self.layers)
            d64 = lambda w: w.detach().double()  # noqa: E731
            f32 = lambda x: x.float().contiguous()  # noqa: E731
            out = {"pq_next": {}, "tables": {}}
            skip64 = d64(self.embedding) @ d64(self.layers[0].Wsc0)
            for t in range(L - 1):
                w1n = d64(self.layers[t + 1].W1)
                ws, wr = w1n[:C, :4 * C], w1n[C:2 * C, :4 * C]
                wo0, wsc0 = d64(self.layers[t].Wo0), d64(self.layers[t].Wsc0)
                if t == 0:
                    bp, bq = f32((wo0 @ ws).t()), f32((wo0 @ wr).t())
                    out["tables"]["p_next"] = f32(skip64 @ ws)
                    out["tables"]["q_next"] = f32(skip64 @ wr)
                else:
                    stack = torch.cat([wo0, wsc0], 0)
                    bp, bq = f32((stack @ ws).t()), f32((stack @ wr).t())
                out["pq_next"][t] = (bp, bq, split_planes(bp), split_planes(bq))
            last = self.layers[L - 1]
            wr2a = d64(self.Wr2a)
            out["y"] = f32((torch.cat([d64(last.Wo0), d64(last.Wsc0)], 0) @ wr2a).t())
            gb, gs = f32(d64(last.Wo0) @ wr2a), f32(d64(last.Wsc0) @ wr2a)
            out["gy"] = (gb, gs)
            out["tables"]["skip"] = f32(skip64)
            hit = (key, out)
            self.__dict__["_merged_cache"] = hit
        return hit[1]

    def first_layer_pq(self) -> tuple[Tensor, Tensor]:
        """The first layer's node-factored blocks per element, embedding @ W1[:C, :2C] and
        embedding @ W1[C:2C, :2C] ([elements, 2C] each; the first layer's input is the embedding,
        so P and Q of an atom depend on its element only), formed in float64 and rounded once;
        rebuilt when either weight changes in place."""
        mats = (self.embedding, self.layers[0].W1)
        key = tuple((w.data_ptr(), w._version, w.device) for w in mats)
        hit = self.__dict__.get("_pq0_cache")
        if hit is None or hit[0] != key:
            C = self.config.channels
            emb, w1 = self.embedding.detach().double(), self.layers[0].W1.detach().double()
            tables = ((emb @ w1[:C, :2 * C]).float().contiguous(), (emb @ w1[C:2 * C, :2 * C]).float().contiguous())
            hit = (key, tables)
            self.__dict__["_pq0_cache"] = hit
        return hit[1]

    def w1_planes(self, t: int, which: str, nz: int = 0) -> Planes:
        """bf16 planes (split once per W1 version) of the weights of layer t's edge GEMMs when the
        operands come pre-split: "receiver" / "sender" / "sender_node" = the first nz rows of
        w1_receiver_t / w1_sender_t / w1_sender_node_t (the forward's [nz, K] B operands)."""
        w = self.layers[t].W1
        key = (w.data_ptr(), w._version, w.device)
        cache = self.__dict__.setdefault("_w1p_cache", {})
        hit = cache.get((t, which, nz))
        if hit is None or hit[0] != key:
            C = self.config.channels
            if which == "receiver":
                src = self.w1_receiver_t(t)[:nz]
            elif which == "sender":
                src = self.w1_sender_t(t)[:nz]
            elif which == "sender_node":
                src = self.w1_sender_node_t(t)[:nz]
            else:
                raise ValueError(f"unknown W1 block {which!r}")
            hit = (key, split_planes(src))
            cache[(t, which, nz)] = hit
        return hit[1]

    def w1_node_blocks(self, t: int) -> Tensor:
        """[W1[:C] | W1[C:2C]] ([C, 8C]): the B operand ([N, K], b_layout 0) of the VJP's node
        GEMM [gzs_src | gzs] @ B^T, the sender and receiver blocks of the gather-cat row gradient;
        rebuilt when W1 is changed in place."""
        w = self.layers[t].W1
        C = self.config.channels
        key = (w.data_ptr(), w._version, w.device)
        cache = self.__dict__.setdefault("_w1nb_cache", {})
        hit = cache.get(t)
        if hit is None or hit[0] != key:
            hit = (key, torch.cat([w.detach()[:C], w.detach()[C:2 * C]], 1).contiguous())
            cache[t] = hit
        return hit[1]

    def w1_node_blocks_planes(self, t: int):
        """The bf16 planes of ``w1_node_blocks(t)`` (split once per weight version)."""
        w = self.w1_node_blocks(t)
        cache = self.__dict__.setdefault("_w1nb_planes", {})
        hit = cache.get(t)
        if hit is None or hit[0] is not w:
            hit = (w, split_planes(w))
            cache[t] = hit
        return hit[1]

    @property
    def num_interactions(self) -> int:
        return self.config.num_interactions


@dataclass
class MaceLikeInput:
    batch: GraphBatch
    elem: Tensor  # int32 [rows] element index of every atom row
    csr_dst: Csr = field(default=None)
    csr_src: Csr = field(default=None)
    # the energy launch's completion counter (uint32 [1], zero between launches): the explicit
    # force path forms the float64 total in that launch's last workgroup
    sum_counter: Tensor = field(default=None)


def _call(name, *args):
    _abi.call(name, *args, _abi.stream_handle())


def _empty(*shape, device, dtype=torch.float32):
    return torch.empty(*shape, dtype=dtype, device=device)


def _atom_order(batch, n: int) -> int | None:
    """Device address of the builder's spatial order of the atoms (``batch.atom_order``, a
    permutation of the n rows) for the message kernels, or None (atom order)."""
    order = getattr(batch, "atom_order", None)
    return None if order is None or order.numel() != n else order.data_ptr()


def _wave_groups(batch, n: int) -> list:
    """The message kernels' launches as ``(order address, atoms, waves per atom)``: the waves per
    atom of a system are chosen by its own atom count, so that a system batched with others sums
    its rows as it does alone. One launch for one system or equal replicas; for a slot union one
    per run of consecutive slots with the same choice, over the slots' range of the spatial order
    (sorted by system first: slot s holds entries [first row, first row + rows) of it)."""
    order = _atom_order(batch, n)
    slots = getattr(batch, "system_slots", ())
    if not slots:
        size = getattr(batch, "max_system_rows", 0) or n
        return [(order, n, 4 if size <= SPLIT_ROWS_MAX_ATOMS else 1)]
    if order is None:
        raise ValueError("a slot union needs the builder's atom order")
    groups: list = []
    end = 0
    for start, rows, atoms in slots:
        wpa = 4 if atoms <= SPLIT_ROWS_MAX_ATOMS else 1
        if start != end:
            raise ValueError("slot union rows must be consecutive")
        if groups and groups[-1][2] == wpa:
            groups[-1][1] += rows
        else:
            groups.append([order + 4 * start, rows, wpa])
        end = start + rows
    if end != n:
        raise ValueError(f"the slots cover {end} rows of {n}")
    return [tuple(g) for g in groups]


def _call_groups(name: str, groups: list, n_at: int, *args) -> None:
    """One ``name`` call per wave group: ``args`` with the atom count at ``n_at``, the order right
    after it and the waves per atom last (placeholders, replaced per group)."""
    for order, count, wpa in groups:
        a = list(args)
        a[n_at], a[n_at + 1], a[-1] = count, order, wpa
        _call(name, *a)


def _gather_edge_rows(h0: Tensor, ef: Tensor, edge_index: Tensor, out: Tensor) -> None:
    """out[e] = [h0[src e] | h0[dst e] | ef[e]] (src = neighbour column 1, dst = centre column 0)."""
    C, nb = h0.shape[1], ef.shape[1]
    rows = out.shape[0]
    col_src = edge_index[:, 1]
    col_dst = edge_index[:, 0]
    _abi.call("fmd_gather_cat_f32", 3, _abi.ptr_array([h0.data_ptr(), h0.data_ptr(), ef.data_ptr()]),
              _abi.ptr_array([col_src.data_ptr(), col_dst.data_ptr(), None]),
              _abi.array(_abi._i64, [edge_index.stride(0), edge_index.stride(0), 1]),
              _abi.array(_abi._i64, [C, C, nb]), _abi.array(_abi._i32, [C, C, nb]), rows, out.data_ptr(),
              out.stride(0), _abi.stream_handle())


def _factored_blocks(model: MaceLike, t: int, h0: Tensor, elem: Tensor, n: int, nz: int, dev) -> tuple:
    """(P, Q) = (h0 W1[:C, :nz], h0 W1[C:2C, :nz]) of layer t ([n, nz] each): the first layer's
    rows from the per-element tables, later layers' by one grouped node GEMM on pre-split weights."""
    P = _empty(n, nz, device=dev)
    Q = _empty(n, nz, device=dev)
    if t == 0:
        tp, tq = model.first_layer_pq()
        if nz != tp.shape[1]:
            raise ValueError("the first layer's pre-activation has the a | b blocks only")
        _call("fmd_embed_f32", elem.data_ptr(), tp.data_ptr(), n, nz, P.data_ptr())
        _call("fmd_embed_f32", elem.data_ptr(), tq.data_ptr(), n, nz, Q.data_ptr())
        return P, Q
    ws, wr = model.w1_sender_node_t(t)[:nz], model.w1_receiver_t(t)[:nz]
    gemm_group([{"a": h0, "b": ws, "b_planes": model.w1_planes(t, "sender_node", nz), "out": P},
                {"a": h0, "b": wr, "b_planes": model.w1_planes(t, "receiver", nz), "out": Q}], b_layout=0)
    return P, Q


class _MaceLikeEnergy(Function):
    """positions -> node energies [rows]; backward: dE/dpos by the VJP kernels."""

    @staticmethod
    def forward(ctx, positions, cell, model: MaceLike, inputs: MaceLikeInput):
        cfg = model.config
        batch = inputs.batch
        dev = positions.device
        C, nb, H = cfg.channels, cfg.n_basis, cfg.readout_hidden
        n = positions.shape[0]
        e_cap = batch.edge_index.shape[0]
        if positions.dtype != torch.float32:
            raise ValueError("the MACE-like model runs in float32")
        positions = positions.detach().contiguous()
        cell = cell.detach().to(torch.float32).contiguous()
        n_edges, off, ei = batch.n_edges, batch.edge_offsets, batch.edge_index
        groups = _wave_groups(batch, n)
        elem = inputs.elem
        inv_avg = 1.0 / cfg.avg_num_neighbors
        geo = _empty(e_cap, 8, device=dev)
        ef = _empty(e_cap, nb, device=dev)
        de = _empty(e_cap, nb, device=dev)
        geo_args = (positions.data_ptr(), cell.data_ptr(), system_rows(batch), ei.data_ptr(),
                    batch.edge_image.data_ptr(), n_edges.data_ptr(), e_cap, float(cfg.cutoff), nb, geo.data_ptr(),
                    ef.data_ptr(), de.data_ptr())
        h1 = None
        saved = []
        h_first = None
        L = len(model.layers)
        factored = FACTORED_Z
        # merged node side (node-factored, unfused, two or more layers): each layer's output GEMM
        # launch also forms the next layer's P and Q (from [B0 | h0] with the products of
        # consecutive weights), the last one the readout's y instead of h0n; the first layer's
        # per-element rows (embedding, its P and Q, the residual table and its next-layer blocks,
        # the prefills of h0n and of the next P and Q) come from one gather launch
        merged = MERGED_NODE and factored and not FUSED_NODE and L >= 2
        h0 = _empty(n, C, device=dev)
        pq_next = None
        if merged:
            mw = model.merged_weights()
            tp, tq = model.first_layer_pq()
            tabs = mw["tables"]
            P = _empty(n, 2 * C, device=dev)
            Q = _empty(n, 2 * C, device=dev)
            h0n_first = _empty(n, C, device=dev)
            pq_next = (_empty(n, 4 * C, device=dev), _empty(n, 4 * C, device=dev))
            rows = [(model.embedding, C, h0), (tp, 2 * C, P), (tq, 2 * C, Q)]
            # the first layer's output rows start from per-element rows (residual, next P and Q):
            # added in the output GEMM's epilogue above the small-system sizes (no prefill written
            # and read back), prefilled here by the same launch below them
            rows_in_epilogue = ROWS_IN_EPILOGUE and n > SMALL_NODE_MAX_ATOMS
            if not rows_in_epilogue:
                rows += [(tabs["skip"], C, h0n_first), (tabs["p_next"], 4 * C, pq_next[0]),
                         (tabs["q_next"], 4 * C, pq_next[1])]
            # the edge geometry and these gathers in one launch
            _call("fmd_edge_geometry_embed_f32", *geo_args, elem.data_ptr(), n, len(rows),
                  _abi.ptr_array([r[0].data_ptr() for r in rows]), _abi.array(_abi._i32, [r[1] for r in rows]),
                  _abi.ptr_array([r[2].data_ptr() for r in rows]))
            z, q = P, Q
        else:
            _call("fmd_edge_geometry_f32", *geo_args)
            _call("fmd_embed_f32", elem.data_ptr(), model.embedding.data_ptr(), n, C, h0.data_ptr())
        y = None
        # On large edge lists the edge GEMMs take pre-split operands: the radial rows once per
        # evaluation here, h0 once per layer, the weights once per version (bitwise the same z as
        # splitting inside the GEMM, without the splitting arithmetic per output tile)
        hoist = e_cap >= HOIST_MIN_ROWS and not factored
        efp = split_planes(ef) if hoist else None
        w1ef_all = [layer.W1[2 * C:] for layer in model.layers]
        for t, layer in enumerate(model.layers):
            last = t == L - 1
            # z = [h0[src] | h0[dst] | ef] @ W1 ([E, 4C]), the gather-cat fused into the edge GEMM's
            # operand load. On large edge lists the receiver block h0[dst] @ W1[C:2C], the same for
            # every row of a centre, is formed once per atom (q, [N, 4C]) and added by the message
            # kernels, and the edge GEMM multiplies [h0[src] | ef] (K = C + nb).
            # Without vector features (h1 = 0, the first layer) wc and wd multiply only zeros: z keeps
            # just its a | b blocks ([E, 2C], the first 2C columns of W1). Node-factored (the
            # default): z = P, q = Q per atom and the kernels add the radial term per row.
            nz = 4 * C if h1 is not None else 2 * C
            if factored:
                if not merged:
                    z, q = _factored_blocks(model, t, h0, elem, n, nz, dev)
                A0 = _empty(n, C, device=dev)
                A1 = _empty(n, 3, C, device=dev)
                _call_groups("fmd_mace_message_f32", groups, 7, z.data_ptr(), q.data_ptr(), geo.data_ptr(),
                             ei.data_ptr(), off.data_ptr(), n_edges.data_ptr(), e_cap, n, None, C, h0.data_ptr(),
                             _abi.ptr(h1), inv_avg, A0.data_ptr(), A1.data_ptr(), 1, ef.data_ptr(),
                             w1ef_all[t].data_ptr(), nb, 0)
            elif hoist:
                h0p = split_planes(h0)
                q = gemm_planes([(h0p, None)], model.w1_planes(t, "receiver", nz), a_planes=True)
                w1p = model.w1_planes(t, "sender", nz)
            else:
                q = None
                parts, w1 = [(h0, ei[:, 1]), (h0, ei[:, 0]), (ef, None)], model.w1_t(t)[:nz]
            if not factored:
                if hoist:
                    z = gemm_planes([(h0p, ei[:, 1]), (efp, None)], w1p, a_planes=True)
                else:
                    z = gemm_gather(parts, w1)
                A0 = _empty(n, C, device=dev)
                A1 = _empty(n, 3, C, device=dev)
                _call_groups("fmd_mace_message_f32", groups, 7, z.data_ptr(), _abi.ptr(q), geo.data_ptr(),
                             ei.data_ptr(), off.data_ptr(), n_edges.data_ptr(), e_cap, n, None, C, h0.data_ptr(),
                             _abi.ptr(h1), inv_avg, A0.data_ptr(), A1.data_ptr(), 0, None, None, 0, 0)
            B0 = _empty(n, C, device=dev)
            B1 = None if last else _empty(n, 3, C, device=dev)
            if FUSED_NODE:
                # the node side of the layer in one launch per 32-atom tile
                w = model.node_weights(t)
                P0 = _empty(n, C, device=dev)
                P1 = _empty(n, 3, C, device=dev)
                h0n = _empty(n, C, device=dev)
                h1n = None if last else _empty(n, 3, C, device=dev)
                _call("fmd_mace_node_fwd_f32", A0.data_ptr(), A1.data_ptr(), h0.data_ptr(), elem.data_ptr(),
                      w["wm0t"].data_ptr(), w["wm1t"].data_ptr(), layer.Wc.data_ptr(), layer.Wd.data_ptr(),
                      w["wout0"].data_ptr(), w["wout1"].data_ptr(), n, C, P0.data_ptr(), P1.data_ptr(),
                      B0.data_ptr(), _abi.ptr(B1), h0n.data_ptr(), _abi.ptr(h1n))
            else:
                # the node side as two grouped GEMM launches around the contraction:
                # (P0 = A0 Wm0, P1 = A1 Wm1), then (h0n = [B0 | h0] [Wo0; Wsc0], h1n = B1 Wo1), with
                # the weights K-contiguous (the split-plane form of a large group)
                w = model.node_weights(t)
                wp = w["planes"]
                P0 = _empty(n, C, device=dev)
                P1 = _empty(n, 3, C, device=dev)
                if n <= SMALL_NODE_MAX_ATOMS:
                    _call("fmd_mace_mix_symcon_f32", A0.data_ptr(), A1.data_ptr(), w["wm0t"].data_ptr(),
                          w["wm1t"].data_ptr(), elem.data_ptr(), layer.Wc.data_ptr(), layer.Wd.data_ptr(), n, C,
                          P0.data_ptr(), P1.data_ptr(), B0.data_ptr(), _abi.ptr(B1))
                else:
                    gemm_group([{"a": A0, "b": w["wm0t"], "b_planes": wp["wm0t"], "out": P0},
                                {"a": A1.view(3 * n, C), "b": w["wm1t"], "b_planes": wp["wm1t"],
                                 "out": P1.view(3 * n, C)}], b_layout=0)
                    _call("fmd_mace_symcon_f32", P0.data_ptr(), P1.data_ptr(), elem.data_ptr(), layer.Wc.data_ptr(),
                          layer.Wd.data_ptr(), n, C, B0.data_ptr(), _abi.ptr(B1))
                h0n = None if merged and last else (h0n_first if merged and t == 0 else _empty(n, C, device=dev))
                h1n = None if last else _empty(n, 3, C, device=dev)
                if merged and last:
                    # the readout's first product from [B0 | h0]: the last layer's h0n is not formed
                    y = _empty(n, H, device=dev)
                    gemm_group([{"a": B0, "a2": h0, "b": mw["y"], "out": y}], b_layout=0)
                elif merged:
                    # h0n, h1n and the next layer's P and Q in one launch (the first layer's h0n and
                    # P, Q prefilled with their per-element residual rows)
                    bp, bq, bpp, bqp = mw["pq_next"][t]
                    P_n, Q_n = pq_next if t == 0 else (_empty(n, 4 * C, device=dev), _empty(n, 4 * C, device=dev))
                    if t == 0:
                        probs = [{"a": B0, "b": w["wo0t"], "b_planes": wp["wo0t"], "out": h0n},
                                 {"a": B0, "b": bp, "b_planes": bpp, "out": P_n},
                                 {"a": B0, "b": bq, "b_planes": bqp, "out": Q_n}]
                        for prob, tab in zip(probs, ("skip", "p_next", "q_next")):
                            if rows_in_epilogue:
                                prob["row_add"] = (tabs[tab], elem)
                            else:
                                prob["accumulate"] = True
                    else:
                        probs = [{"a": B0, "a2": h0, "b": w["wout0"], "b_planes": wp["wout0"], "out": h0n},
                                 {"a": B0, "a2": h0, "b": bp, "b_planes": bpp, "out": P_n},
                                 {"a": B0, "a2": h0, "b": bq, "b_planes": bqp, "out": Q_n}]
                    probs.append({"a": B1.view(3 * n, C), "b": w["wo1t"], "b_planes": wp["wo1t"],
                                  "out": h1n.view(3 * n, C)})
                    gemm_group(probs, b_layout=0)
                elif t == 0:
                    # h0 is the embedding: the residual h0 Wsc0 is a per-element table (rounded
                    # once), added to B0 Wo0 in the GEMM's epilogue
                    _call("fmd_embed_f32", elem.data_ptr(), model.skip_table().data_ptr(), n, C, h0n.data_ptr())
                    probs = [{"a": B0, "b": w["wo0t"], "b_planes": wp["wo0t"], "out": h0n, "accumulate": True}]
                else:
                    probs = [{"a": B0, "a2": h0, "b": w["wout0"], "b_planes": wp["wout0"], "out": h0n}]
                if not merged:
                    if not last:
                        probs.append({"a": B1.view(3 * n, C), "b": w["wo1t"], "b_planes": wp["wo1t"],
                                      "out": h1n.view(3 * n, C)})
                    gemm_group(probs, b_layout=0)
            saved.append((h0, h1, z, q, P0, P1))
            if t == 0:
                h_first = h0n
            if merged and not last:
                z, q = P_n, Q_n
            h0, h1 = h0n, h1n
        if y is None:
            y = gemm(h0, model.Wr2a, b_layout=1)  # [N, H]
        energy = _empty(n, device=dev)
        if getattr(ctx, "seed_ones", False):
            # the explicit force path (seed dE/dE_i = 1): the readout's gradients in the same launch
            ctx.gha, ctx.gy = _empty(n, C, device=dev), _empty(n, H, device=dev)
            total = getattr(ctx, "total", None)
            _call("fmd_mace_energy_grad_f32", h_first.data_ptr(), model.wr1.data_ptr(), y.data_ptr(),
                  model.wr2b.data_ptr(), C, H, elem.data_ptr(), model.e0.data_ptr(), float(cfg.scale),
                  float(cfg.shift), n, energy.data_ptr(), ctx.gha.data_ptr(), ctx.gy.data_ptr(), _abi.ptr(total),
                  _abi.ptr(inputs.sum_counter if total is not None else None))
        else:
            _call("fmd_mace_energy_f32", h_first.data_ptr(), model.wr1.data_ptr(), y.data_ptr(),
                  model.wr2b.data_ptr(), C, H, elem.data_ptr(), model.e0.data_ptr(), float(cfg.scale),
                  float(cfg.shift), n, energy.data_ptr())
        ctx.model, ctx.inputs, ctx.saved = model, inputs, saved
        ctx.geo, ctx.de, ctx.y, ctx.ef, ctx.factored, ctx.merged = geo, de, y, ef, factored, merged
        ctx.n, ctx.e_cap = n, e_cap
        return energy

    @staticmethod
    def backward(ctx, gE):
        gE = gE.detach().to(torch.float32).contiguous()
        return _vjp(ctx, gE, 1.0), None, None, None


class _Saved:
    """What the forward keeps for the VJP (the autograd ctx, or this holder outside autograd). The
    explicit force path seeds dE/dE_i = 1, so its forward also forms the readout's gradients."""

    seed_ones = True


def _vjp(ctx, gE: Tensor | None, sign: float, stress_cell: Tensor | None = None):
    """``sign * dE/dpos`` [rows, 3] with E = sum_i gE_i E_i (gE None: all ones), by the VJP kernels;
    with ``stress_cell`` (the unstrained float32 cell) also the stress dE/d(strain) / V [3, 3]:
    ``(forces, stress)``."""
    model, inputs = ctx.model, ctx.inputs
    cfg = model.config
    batch = inputs.batch
    C, nb, H = cfg.channels, cfg.n_basis, cfg.readout_hidden
    n, e_cap = ctx.n, ctx.e_cap
    dev = ctx.geo.device
    inv_avg = 1.0 / cfg.avg_num_neighbors
    n_edges, off, ei, rev = batch.n_edges, batch.edge_offsets, batch.edge_index, batch.edge_reverse
    groups = _wave_groups(batch, n)
    # readouts: gha = dE/d(first layer's h0 out), gy -> dE/d(last layer's h0 out)
    if gE is None and getattr(ctx, "gha", None) is not None:
        gha, gy = ctx.gha, ctx.gy  # formed by the forward's energy launch
    else:
        gy = _empty(n, H, device=dev)
        gha = _empty(n, C, device=dev)
        _call("fmd_mace_energy_bwd_f32", _abi.ptr(gE), model.wr1.data_ptr(), ctx.y.data_ptr(),
              model.wr2b.data_ptr(), C, H, float(cfg.scale), n, gha.data_ptr(), gy.data_ptr())
    # dE/dh0 out of the last layer (with one layer, the first readout's gradient joins here)
    L = len(model.layers)
    # merged: the last layer's h0n was never formed; its VJP's first products start from gy
    g_out0 = None if ctx.merged else gemm(gy, model.Wr2a, b_layout=0, out=gha if L == 1 else None,
                                          accumulate=L == 1)
    g_out1 = None  # dE/dh1 out of the current layer (the last layer's h1 out is unused)
    ggeo = _empty(e_cap, 4, device=dev)
    gefs = []
    for t in reversed(range(L)):
        layer = model.layers[t]
        h0, h1, z, q, P0, P1 = ctx.saved[t]
        gP0 = _empty(n, C, device=dev)
        gP1 = _empty(n, 3, C, device=dev)
        g_in0 = None
        if FUSED_NODE:
            # node side of the layer's VJP in one launch per 32-atom tile; with t > 0 it also forms
            # this layer's input gradient through the residual, g_in0 = g_out0 Wsc0^T (added to the
            # first readout's gradient in the second layer)
            w = model.node_weights(t)
            gB0 = _empty(n, C, device=dev)
            gB1 = None if g_out1 is None else _empty(n, 3, C, device=dev)
            gA0 = _empty(n, C, device=dev)
            gA1 = _empty(n, 3, C, device=dev)
            if t > 0:
                g_in0 = gha if t == 1 else _empty(n, C, device=dev)
            _call("fmd_mace_node_bwd_f32", g_out0.data_ptr(), _abi.ptr(g_out1), P0.data_ptr(), P1.data_ptr(),
                  inputs.elem.data_ptr(), w["wo0st"].data_ptr(), w["wo1st"].data_ptr(), layer.Wc.data_ptr(),
                  layer.Wd.data_ptr(), layer.Wm0.data_ptr(), layer.Wm1.data_ptr(), n, C, gB0.data_ptr(),
                  _abi.ptr(gB1), _abi.ptr(g_in0), 1 if t == 1 else 0, gP0.data_ptr(), gP1.data_ptr(),
                  gA0.data_ptr(), gA1.data_ptr())
        else:
            # gB0 = g_out0 Wo0^T, gB1 = g_out1 Wo1^T, the contraction's VJP (gP0, gP1), then
            # gA0 = gP0 Wm0^T, gA1 = gP1 Wm1^T; with t > 0 also this layer's input gradient through
            # the residual, g_in0 = g_out0 Wsc0^T, added to the first readout's gradient in the second
            # layer. Small launches: the first three in one kernel, g_in0 in the gA group; else
            # grouped GEMM launches around the contraction's VJP kernel, g_in0 in the first group.
            wp = model.node_weights(t)["planes"]
            gA0 = _empty(n, C, device=dev)
            gA1 = _empty(n, 3, C, device=dev)
            gA_probs = [{"a": gP0, "b": layer.Wm0, "b_planes": wp["Wm0"], "out": gA0},
                        {"a": gP1.view(3 * n, C), "b": layer.Wm1, "b_planes": wp["Wm1"], "out": gA1.view(3 * n, C)}]
            if g_out0 is None:
                # the last layer under the merged node side: gB0 = gy (Wo0 Wr2a)^T and the residual's
                # g_in0 = gy (Wsc0 Wr2a)^T (gy [N, H]: K = H)
                gb, gs = model.merged_weights()["gy"]
                g0, wb0, k0, ws, wsp = gy, gb, H, gs, None
            else:
                g0, wb0, k0, ws, wsp = g_out0, layer.Wo0, C, layer.Wsc0, wp["Wsc0"]
            if t > 0:
                g_in0 = gha if t == 1 else _empty(n, C, device=dev)
                res = {"a": g0, "b": ws, "out": g_in0, "accumulate": t == 1}
                if wsp is not None:
                    res["b_planes"] = wsp
            if n <= SMALL_NODE_MAX_ATOMS:
                # gB0, gB1 and the contraction's VJP in one launch; the residual's input gradient
                # joins the gA group
                _call("fmd_mace_mix_symcon_bwd_f32", g0.data_ptr(), k0, wb0.data_ptr(), _abi.ptr(g_out1),
                      layer.Wo1.data_ptr(), P0.data_ptr(), P1.data_ptr(), inputs.elem.data_ptr(), layer.Wc.data_ptr(),
                      layer.Wd.data_ptr(), n, C, gP0.data_ptr(), gP1.data_ptr())
                gemm_group(gA_probs + ([res] if t > 0 else []), b_layout=0)
            else:
                gB0 = _empty(n, C, device=dev)
                gB1 = None if g_out1 is None else _empty(n, 3, C, device=dev)
                probs = [{"a": g0, "b": wb0, "out": gB0}]
                if g_out0 is not None:
                    probs[0]["b_planes"] = wp["Wo0"]
                if gB1 is not None:
                    probs.append({"a": g_out1.reshape(3 * n, C), "b": layer.Wo1, "b_planes": wp["Wo1"],
                                  "out": gB1.view(3 * n, C)})
                if t > 0:
                    probs.append(res)
                gemm_group(probs, b_layout=0)
                _call("fmd_mace_symcon_bwd_f32", P0.data_ptr(), P1.data_ptr(), inputs.elem.data_ptr(),
                      layer.Wc.data_ptr(), layer.Wd.data_ptr(), gB0.data_ptr(), _abi.ptr(gB1), n, C, gP0.data_ptr(),
                      gP1.data_ptr())
                gemm_group(gA_probs, b_layout=0)
        acc_geo = 1 if t < L - 1 else 0
        if t == 0:
            # the first layer's inputs are the element embedding (no position dependence): only
            # the radial-basis block of its gather-cat row gradient is needed, formed in the
            # kernel from W1's radial rows (gz is not stored)
            gef = _empty(e_cap, nb, device=dev)
            w1ef = layer.W1[2 * C:]
            _call_groups("fmd_mace_message_bwd_f32", groups, 8, z.data_ptr(), _abi.ptr(q), ctx.geo.data_ptr(),
                         ei.data_ptr(), rev.data_ptr(), off.data_ptr(), n_edges.data_ptr(), e_cap, n, None, C,
                         h0.data_ptr(), _abi.ptr(h1), gA0.data_ptr(), gA1.data_ptr(), inv_avg, None, None, None,
                         ggeo.data_ptr(), acc_geo, None, None, 0, w1ef.data_ptr(), nb, gef.data_ptr(),
                         1 if ctx.factored else 0, ctx.ef.data_ptr(), 0)
            gefs.append((gef, nb))
            break
        # the gather-cat row gradient's node blocks come from per-node sums of g_z (never stored):
        # over each centre's rows (receiver, gzs) and over each sender's rows (gzs_src, formed by
        # the sender-side kernel); by linearity sum_e g_z[e] W^T = (sum_e g_z[e]) W^T
        gzs = _empty(n, 4 * C, device=dev)
        gzs_src = _empty(n, 4 * C, device=dev)
        gef = _empty(e_cap, nb, device=dev)
        # this layer's inputs: residual (plus, in the second layer, the first readout's
        # gradient of the first layer's output), sender side of the messages, gather-cat rows
        if g_in0 is None:
            g_in0 = gemm(g_out0, layer.Wsc0, b_layout=0, out=gha if t == 1 else None, accumulate=t == 1)
        g_in1 = _empty(n, 3, C, device=dev) if h1 is not None else None
        w1ef = layer.W1[2 * C:]
        head = (z.data_ptr(), _abi.ptr(q), ctx.geo.data_ptr(), ei.data_ptr(), rev.data_ptr(), off.data_ptr(),
                n_edges.data_ptr(), e_cap, n, None, C, h0.data_ptr(), _abi.ptr(h1), gA0.data_ptr(), gA1.data_ptr(),
                inv_avg, None, gzs.data_ptr())
        tail = (w1ef.data_ptr(), nb, gef.data_ptr(), 1 if ctx.factored else 0, ctx.ef.data_ptr(), 0)
        _call_groups("fmd_mace_message_bwd_f32", groups, 8, *head, gzs_src.data_ptr(), ggeo.data_ptr(), acc_geo,
                     g_in0.data_ptr(), _abi.ptr(g_in1), 1, *tail)
        # g_in0 += [gzs_src | gzs] [W1[:C] | W1[C:2C]]^T (sender and receiver blocks, one node GEMM)
        # (as four K slices of one split-plane group, the weights split once: 20 us per step less at
        # 10 000 atoms than eight fp32 MFMA slices)
        gemm_splitk(gzs_src, model.w1_node_blocks(t), b_layout=0, out=g_in0, a2=gzs, accumulate=True,
                    b_planes=model.w1_node_blocks_planes(t))
        gefs.append((gef, nb))
        g_out0, g_out1 = g_in0, g_in1
    gvec = _empty(e_cap, 3, device=dev)
    (g0, ld0) = gefs[0]
    (g1, ld1) = gefs[1] if len(gefs) > 1 else (None, 0)
    _call("fmd_edge_geometry_bwd_f32", ctx.geo.data_ptr(), ctx.de.data_ptr(), nb, g0.data_ptr(), ld0,
          _abi.ptr(g1), ld1, ggeo.data_ptr(), n_edges.data_ptr(), e_cap, gvec.data_ptr())
    forces = segment_sum_csr([(gvec, inputs.csr_src, 0, sign, None), (gvec, inputs.csr_dst, 0, -sign, None)], n, 3)
    if stress_cell is None:
        return forces
    from fastmd_amd.engine.energy_derivative import edge_stress

    return forces, edge_stress(ctx.geo, gvec, n_edges, stress_cell)


class MaceLikeAdapter:
    """The MACE-like model as a ModelAdapter with an EnergyTap (mace.py:254-477's surface)."""

    name = "mace_like"
    compiled = False

    def __init__(self, module: MaceLike | None = None, *, config: MaceLikeConfig | None = None,
                 device: torch.device | str = "cuda") -> None:
        module = module if module is not None else MaceLike(config or MaceLikeConfig())
        self.module = module.to(device).eval()
        for p in self.module.parameters():
            p.requires_grad_(False)

    def topology_spec(self) -> TopologySpec:
        cfg = self.module.config
        return TopologySpec(cutoff=float(cfg.cutoff), num_interactions=int(cfg.num_interactions),
                            model_dtype="float32", edge_order="sorted")

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

    def prepare(self, batch: GraphBatch) -> MaceLikeInput:
        """Aliases of the batch plus the element index of every row (host check of the species,
        outside any graph) and the two CSRs of the edge list."""
        if batch.positions is None or batch.edge_offsets is None or batch.edge_reverse is None:
            raise ValueError("the MACE-like model needs an edges-only batch with its CSR (edge_offsets, edge_reverse)")
        require_atom_rows(batch, "MACE-like")
        species = batch.species.long()
        table = self.module.z_table.to(species.device)
        if bool(((species < 1) | (species > _ELEMENTS)).any()) or bool((table[species.clamp(1, _ELEMENTS)] < 0).any()):
            raise ValueError(f"the MACE-like model supports atomic numbers {list(self.module.config.elements)}")
        elem = table[species].to(torch.int32).contiguous()
        rows = batch.edge_index.shape[0]
        return MaceLikeInput(batch=batch, elem=elem, csr_dst=Csr(batch.edge_offsets, None, rows),
                             csr_src=Csr(batch.edge_offsets, batch.edge_reverse, rows),
                             sum_counter=torch.zeros(1, dtype=torch.int32, device=elem.device))

    def node_energy(self, inputs: MaceLikeInput, positions: Tensor, cell: Tensor) -> Tensor:
        """Per-atom energies [rows] (float32) at ``positions``; differentiable w.r.t. positions."""
        if cell.requires_grad:
            raise NotImplementedError("stress (a strained cell) is not supported by the MACE-like kernels")
        return _MaceLikeEnergy.apply(positions, cell, self.module, inputs)

    def energy_and_forces(self, inputs: MaceLikeInput, positions: Tensor, cell: Tensor,
                          segments=1) -> tuple[Tensor, Tensor]:
        """(E [1] float64 = the fixed-order sum of the node energies, F = -dE/dpos [rows, 3]) without
        autograd: the same forward and VJP kernels as ``node_energy`` + ``torch.autograd.grad``, minus
        the autograd seed, cast and negation kernels."""
        from fastmd_amd.engine.energy_derivative import sum_f64_segments

        saved = _Saved()
        # (small launches only: each of the energy launch's blocks fences at device scope)
        one = (isinstance(segments, int) and segments == 1 and inputs.sum_counter is not None
               and positions.shape[0] <= ENERGY_TOTAL_MAX_ATOMS)
        if one:
            # the fixed-order total of all rows, formed by the energy launch itself
            saved.total = torch.empty(1, dtype=torch.float64, device=positions.device)
        energies = _MaceLikeEnergy.forward(saved, positions.detach(), cell.detach(), self.module, inputs)
        # one energy per replica or system
        energy = saved.total if one else sum_f64_segments(energies, segments)
        return energy, _vjp(saved, None, -1.0)

    def energy_forces_stress(self, inputs: MaceLikeInput, positions: Tensor, cell: Tensor):
        """``energy_and_forces`` plus the stress dE/d(strain) / V [3, 3] float32 of one system
        (energy_derivative.py:110-140), from the same VJP's edge-vector gradient."""
        from fastmd_amd.engine.energy_derivative import sum_f64_into

        saved = _Saved()
        energies = _MaceLikeEnergy.forward(saved, positions.detach(), cell.detach(), self.module, inputs)
        energy = sum_f64_into(energies)
        forces, stress = _vjp(saved, None, -1.0, stress_cell=cell.detach().to(torch.float32).contiguous())
        return energy, forces, stress
