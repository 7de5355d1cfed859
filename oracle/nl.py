"""Neighbour-list oracle (test infrastructure only; see oracle/__init__.py).

Restates, in NumPy float32 with the operation order of ``fastmd_amd/csrc/nl.hip``:
  * the wrap of FixedCapacityGraphBuilder.build / refresh_candidates
    (fastmd/graph/fixed_capacity_builder.py:1674-1685, 2199-2252; small_matmul geometry.py:7-34)
  * the candidate list of the cell-list refresh (nvalchemiops' role at
    fixed_capacity_builder.py:1519-1554), as the full set of (j, shift) within the candidate
    cutoff, sorted by (j, sx, sy, sz), first bmax stored, all counted
  * _count_neighbors_kernel / _materialize_neighbors_kernel (:97-288), the exclusive scan
    (:1814-1815), far self-loop padding (_pad_self_loops_kernel :323-366, self_loop_padding
    :1004-1027), sink padding (_pad_edges_kernel :291-320), the exact-cutoff override
    (HAS_OVERRIDE, :357-361), the canonical sort (_sort_edges :1968-1999) and the overflow flag
  * fixed_capacity_exceeded (:796-814) and the window flag fold (:430-455)
  * the three-body line graph: the short-bond flags of the materialization (:258-260), the
    undirected pairs of _materialize_pairs (:2001-2084), the short lists, pair offsets and
    overflow rule of _materialize_line_graph (:2086-2161) and the triplet rows of
    _line_graph_kernel (:680-753), far self-loop padding (LOOP_PADDING) or sink padding, with
    the all-loop / all-sink overflow topology of _allocate_overflow_topology (:1474-1513) and
    its edge rows (_substitute_overflow_topology :2163-2177)
  * estimate_max_neighbors (fastmd/graph/neighbor_list_backend.py:77-88) and the ragged
    builder's slot growth rule (fastmd/graph/gpu_graph_builder.py:74-85)
and an FP64 brute-force pair set (tests/test_fixed_capacity_boundary.py:86-102) that pins it.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

F32 = np.float32


def estimate_max_neighbors(cutoff: float, atomic_density: float = 0.35, safety_factor: float = 5.0) -> int:
    """neighbor_list_backend.py:77-88."""
    if cutoff <= 0:
        return 0
    volume = atomic_density * (4.0 / 3.0) * math.pi * (cutoff ** 3)
    expected = max(1, safety_factor * volume)
    return int(math.ceil(expected / 16)) * 16


def grown_max_neighbors(capacity: int, max_count: int, quantum: int = 16) -> int:
    """gpu_graph_builder.py:83-85."""
    return max(2 * capacity, -(-max_count // quantum) * quantum)


def wrap(positions, inv_cell, cell):
    """(frac, wraps, wrapped) in float32 (nl.hip wrap_position)."""
    x = np.asarray(positions).astype(F32)
    inv = np.asarray(inv_cell, dtype=F32)
    c = np.asarray(cell, dtype=F32)
    t = x[:, 0:1] * inv[0]
    t = t + x[:, 1:2] * inv[1]
    t = t + x[:, 2:3] * inv[2]
    fl = np.floor(t)
    wraps = fl.astype(np.int32)
    frac = (t - fl).astype(F32)
    w = frac[:, 0:1] * c[0]
    w = w + frac[:, 1:2] * c[1]
    w = w + frac[:, 2:3] * c[2]
    return frac, wraps, w.astype(F32)


def pair_d2(pi, pj, img, cell):
    """float32 squared distance of rows pi -> pj + img @ cell in nl.hip's order; returns (d2, d)."""
    c = np.asarray(cell, dtype=F32)
    s = np.asarray(img).astype(F32)
    d = []
    for k in range(3):
        v = pj[:, k] - pi[:, k]
        v = v + s[:, 0] * c[0, k]
        v = v + s[:, 1] * c[1, k]
        v = v + s[:, 2] * c[2, k]
        d.append(v.astype(F32))
    d2 = d[0] * d[0]
    d2 = d2 + d[1] * d[1]
    d2 = d2 + d[2] * d[2]
    return d2.astype(F32), np.stack(d, 1)


def cell_heights(cell) -> np.ndarray:
    c = np.asarray(cell, dtype=np.float64)
    volume = abs(np.linalg.det(c))
    return np.array([volume / np.linalg.norm(np.cross(c[(k + 1) % 3], c[(k + 2) % 3])) for k in range(3)])


def _candidate_pairs(wrapped, cell, cutoff):
    """A superset of the directed (i, j, shift) pairs within `cutoff` (float64 search)."""
    n = wrapped.shape[0]
    reach = [int(math.ceil(cutoff / h)) + 1 for h in cell_heights(cell)]
    images = np.array(np.meshgrid(*[np.arange(-r, r + 1) for r in reach], indexing="ij")).reshape(3, -1).T
    pos = wrapped.astype(np.float64)
    cell64 = np.asarray(cell, dtype=np.float64)
    margin = cutoff + 0.05
    out_i, out_j, out_s = [], [], []
    if n * n * len(images) <= 4_000_000:
        for s in images:
            v = pos[None, :, :] + (s @ cell64)[None, None, :] - pos[:, None, :]
            d = np.sqrt((v * v).sum(-1))
            ii, jj = np.nonzero(d < margin)
            out_i.append(ii)
            out_j.append(jj)
            out_s.append(np.broadcast_to(s, (ii.size, 3)))
    else:
        from scipy.spatial import cKDTree

        tree = cKDTree(pos)
        for s in images:
            shifted = pos + s @ cell64
            pairs = cKDTree(shifted).query_ball_tree(tree, margin)  # pairs[j] = atoms i near image j
            jj = np.repeat(np.arange(n), [len(p) for p in pairs])
            ii = np.fromiter((i for p in pairs for i in p), dtype=np.int64, count=jj.size)
            out_i.append(ii)
            out_j.append(jj)
            out_s.append(np.broadcast_to(s, (ii.size, 3)))
    i = np.concatenate(out_i).astype(np.int64)
    j = np.concatenate(out_j).astype(np.int64)
    s = np.concatenate(out_s).astype(np.int32)
    return i, j, s


@dataclass
class Candidates:
    neighbor_matrix: np.ndarray  # int32 [n, bmax], pad n
    neighbor_shifts: np.ndarray  # int32 [n, bmax, 3]
    num_neighbors: np.ndarray  # int32 [n]
    capacity_valid: bool


def candidates(wrapped, cell, cutoff2, bmax: int) -> Candidates:
    """The refresh's candidate rows (see module docstring); `wrapped` are the wrapped float32
    coordinates, `cutoff2` the float32 square of the candidate cutoff."""
    wrapped = np.asarray(wrapped, dtype=F32)
    n = wrapped.shape[0]
    cutoff2 = F32(cutoff2)
    i, j, s = _candidate_pairs(wrapped, cell, float(np.sqrt(np.float64(cutoff2))))
    d2, _ = pair_d2(wrapped[i], wrapped[j], s, cell)
    keep = (d2 < cutoff2) & ~((i == j) & (s == 0).all(1))
    i, j, s = i[keep], j[keep], s[keep]
    order = np.lexsort((s[:, 2], s[:, 1], s[:, 0], j, i))
    i, j, s = i[order], j[order], s[order]
    counts = np.bincount(i, minlength=n).astype(np.int32)
    starts = np.concatenate([[0], np.cumsum(counts)])
    rank = np.arange(i.size) - starts[i]
    stored = rank < bmax
    nm = np.full((n, bmax), n, dtype=np.int32)
    ns = np.zeros((n, bmax, 3), dtype=np.int32)
    nm[i[stored], rank[stored]] = j[stored]
    ns[i[stored], rank[stored]] = s[stored]
    return Candidates(nm, ns, counts, bool((counts <= bmax).all()))


def self_loop_image(cell, cutoff: float, min_length: float = 0.0):
    """Far self-loop padding image and length (fixed_capacity_builder.py:1004-1027)."""
    lengths = np.linalg.norm(np.asarray(cell, dtype=np.float64), axis=1)
    axis = int(np.argmax(lengths))
    longest = float(lengths[axis])
    if not longest > 0.0:
        raise ValueError("far self-loop padding needs a cell with a nonzero lattice vector")
    multiple = max(1, math.ceil(max(min_length, 2.0 * cutoff) / longest))
    image = [0, 0, 0]
    image[axis] = multiple
    return tuple(image), multiple * longest


@dataclass
class Build:
    frac: np.ndarray
    wrap_delta: np.ndarray
    wrapped: np.ndarray
    edge_counts: np.ndarray  # int64 [n]
    edge_offsets: np.ndarray  # int64 [n+1]
    center: np.ndarray  # int32 [e_cap]
    neighbor: np.ndarray
    images: np.ndarray  # int32 [e_cap, 3]
    distances: np.ndarray  # float32 [e_cap] (rows >= real rows undefined: NaN here)
    max_displacement: np.float32
    candidate_valid: bool
    overflow: bool
    isolated: int
    short: np.ndarray | None = None  # bool [e_cap]: real rows with d2 < line2 (line-graph builds)

    @property
    def n_edges(self) -> int:
        return int(self.edge_offsets[-1])


def build(positions, inv_cell, cell, cand: Candidates, reference_positions, reference_wraps, rc2, skin_limit,
          pad_image, e_cap: int, line2: float | None = None, minimum_image: bool = False, n_dummy: int = 0) -> Build:
    """One build over the candidate list (see module docstring); with ``line2`` (the float32
    square of the bond cutoff) also the short-bond flag of every row. ``n_dummy`` > 0: sink
    padding (padded row r on sink n + p n_dummy // max(e_cap // 2 - ec // 2, 1), p = (r - ec) // 2,
    image (3, 3, 3), distance 1e6); otherwise far self-loops with ``pad_image``. ``minimum_image``
    (fixed_capacity_builder.py:2233-2245): a lattice jump since the refresh is no motion; the
    displacement d loses jumps = round(d @ inv_cell) (float32, half to even) times the cell, and
    the jumps leave the wrap delta."""
    pos = np.asarray(positions).astype(F32)
    n = pos.shape[0]
    frac, wraps, wrapped = wrap(pos, inv_cell, cell)
    wd = (wraps - np.asarray(reference_wraps, dtype=np.int32)).astype(np.int32)
    disp = pos - np.asarray(reference_positions, dtype=F32)
    if minimum_image:
        inv = np.asarray(inv_cell, dtype=F32)
        c = np.asarray(cell, dtype=F32)
        t = disp[:, 0:1] * inv[0]
        t = t + disp[:, 1:2] * inv[1]
        t = t + disp[:, 2:3] * inv[2]
        jumps = np.rint(t).astype(F32)
        m = jumps[:, 0:1] * c[0]
        m = m + jumps[:, 1:2] * c[1]
        m = m + jumps[:, 2:3] * c[2]
        disp = (disp - m).astype(F32)
        wd = (wd - jumps.astype(np.int32)).astype(np.int32)
    s = disp[:, 0] * disp[:, 0]
    s = s + disp[:, 1] * disp[:, 1]
    s = s + disp[:, 2] * disp[:, 2]
    norms = np.sqrt(s.astype(F32))
    max_disp = F32(np.max(norms)) if n else F32(0)
    valid = bool((max_disp * F32(2.0) <= F32(skin_limit)) and cand.capacity_valid)

    bmax = cand.neighbor_matrix.shape[1]
    cnt = np.minimum(cand.num_neighbors, bmax)
    slot = np.arange(bmax)[None, :] < cnt[:, None]
    ii, ss = np.nonzero(slot)  # row-major: ascending (atom, slot)
    jj = np.minimum(cand.neighbor_matrix[ii, ss], n - 1)
    img = cand.neighbor_shifts[ii, ss] + wd[jj] - wd[ii]
    d2, _ = pair_d2(wrapped[ii], wrapped[jj], img, cell)
    edge = d2 < F32(rc2)
    ii, jj, img, d2 = ii[edge], jj[edge], img[edge], d2[edge]
    counts = np.bincount(ii, minlength=n).astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    total = int(offsets[-1])
    ec = min(total, e_cap)
    center = np.empty(e_cap, np.int32)
    neighbor = np.empty(e_cap, np.int32)
    images = np.empty((e_cap, 3), np.int32)
    distances = np.full(e_cap, np.nan, F32)
    center[:ec] = ii[:ec]
    neighbor[:ec] = jj[:ec]
    images[:ec] = img[:ec]
    distances[:ec] = np.sqrt(d2[:ec])
    pad = np.arange(ec, e_cap)
    if n_dummy > 0:
        pair = (pad - ec) // 2
        atoms = (n + pair * n_dummy // max(e_cap // 2 - ec // 2, 1)).astype(np.int32)
        images[ec:] = 3
        distances[ec:] = F32(1.0e6)
    else:
        atoms = ((pad - ec) % n).astype(np.int32)
        images[ec:] = np.asarray(pad_image, dtype=np.int32)
    center[ec:] = atoms
    neighbor[ec:] = atoms
    short = None
    if line2 is not None:
        short = np.zeros(e_cap, bool)
        short[:ec] = d2[:ec] < F32(line2)
    return Build(frac, wd, wrapped, counts, offsets, center, neighbor, images, distances, max_disp, valid,
                 bool(total > e_cap or not valid), int((counts == 0).sum()), short)


def pad_override(n_edges: int, e_cap: int, vector) -> np.ndarray:
    """The exact-cutoff padding's edge-vector override [e_cap, 3] float32: ``vector`` on the padded
    rows [min(n_edges, e_cap), e_cap), 0 on the real rows (fixed_capacity_builder.py:357-361)."""
    out = np.zeros((e_cap, 3), F32)
    out[min(n_edges, e_cap):] = np.asarray(vector, dtype=F32)
    return out


def line_graph(b: Build, rev, n: int, e_cap: int, u_cap: int, t_cap: int, bmax: int, n_dummy: int = 0,
               pad_image=(0, 0, 0)) -> dict:
    """The line graph of a build (module docstring): d2u, u2d, invalid_pairs, short_counts,
    short_offsets, short_edge_matrix, pair_offsets, overflow and the triplet rows; with
    ``n_dummy`` > 0 sink padding. Also the published edge rows center / neighbor / images: the
    build's, or on overflow the all-padding rows (row e on pair e // 2's loop atom or sink, image
    +/- ``pad_image`` or +/- (3, 3, 3) for even / odd e)."""
    total = b.n_edges
    ec = min(total, e_cap)
    ids = np.arange(e_cap, dtype=np.int64)
    rev = np.asarray(rev, dtype=np.int64)
    real = ids < ec
    matched = real & (rev >= 0)
    leader = matched & (ids <= rev)
    canon = np.where(matched & (rev < ids), rev, ids)
    prefix = np.cumsum(leader.astype(np.int64))
    real_u = ec // 2
    d2u = np.where(real, prefix[canon] - 1, real_u + np.maximum(ids - ec, 0) // 2)
    d2u = np.clip(d2u, 0, u_cap - 1)
    u2d = np.full(u_cap, e_cap - 1, np.int64)
    lead_ids = (prefix - 1)[leader]
    ok = (lead_ids >= 0) & (lead_ids < u_cap)
    u2d[lead_ids[ok]] = np.minimum(ids[leader][ok], e_cap - 1)
    u = np.arange(u_cap)
    u2d = np.where(u >= real_u, np.minimum(ec + 2 * (u - real_u), e_cap - 1), u2d)
    invalid = bool(total % 2 != 0 or int(leader.sum()) != total // 2 or bool((real & ~matched).any()))
    short = b.short & real
    s = np.bincount(b.center[short], minlength=n).astype(np.int64)
    short_offsets = np.concatenate([[0], np.cumsum(s)]).astype(np.int64)
    sem = np.full((n, bmax), e_cap, np.int64)
    rows = np.nonzero(short)[0]
    for i in range(n):
        mine = rows[b.center[rows] == i][:bmax]
        sem[i, :len(mine)] = mine
    pair_offsets = np.concatenate([[0], np.cumsum(s * (s - 1))]).astype(np.int64)
    overflow = bool(total >= e_cap or pair_offsets[-1] > t_cap or invalid or not b.candidate_valid)
    lg = np.zeros((t_cap, 5), np.int64)
    t_ids = np.arange(t_cap, dtype=np.int64)
    def overflow_atom(pair):
        return n + pair * n_dummy // u_cap if n_dummy > 0 else pair % n

    center, neighbor, images = b.center.copy(), b.neighbor.copy(), b.images.copy()
    if overflow:
        if n_dummy > 0:
            lu = (t_ids * n_dummy // t_cap * u_cap + n_dummy - 1) // n_dummy
        else:
            lu = t_ids * u_cap // t_cap
        lu = np.minimum(lu, u_cap - 1)
        lg[:] = np.stack([overflow_atom(lu), lu, 2 * lu, lu, 2 * lu], 1)
        d2u = ids // 2
        u2d = 2 * u
        center[:] = neighbor[:] = overflow_atom(ids // 2)
        sign = np.where(ids % 2 == 0, 1, -1)[:, None]
        images[:] = sign * (np.full(3, 3) if n_dummy > 0 else np.asarray(pad_image, dtype=np.int64))
    else:
        t_real = min(int(pair_offsets[-1]), t_cap)
        tr = t_ids[:t_real]
        atom = np.searchsorted(pair_offsets, tr, side="right") - 1
        atom = np.minimum(atom, n - 1)
        local = tr - pair_offsets[atom]
        denom = np.maximum(s[atom] - 1, 1)
        first = local // denom
        second_raw = local - first * denom
        second = second_raw + (second_raw >= first)
        de1 = sem[atom, np.minimum(first, bmax - 1)]
        de2 = sem[atom, np.minimum(second, bmax - 1)]
        lg[:t_real] = np.stack([atom, d2u[np.clip(de1, 0, e_cap - 1)], de1, d2u[np.clip(de2, 0, e_cap - 1)], de2], 1)
        pad_id = t_ids[t_real:] - t_real
        pad_pair = pad_id % max(u_cap - real_u, 1)
        pu, pde = real_u + pad_pair, ec + 2 * pad_pair
        pad_atom = n + pad_id * n_dummy // max(t_cap - t_real, 1) if n_dummy > 0 else pad_pair % n
        lg[t_real:] = np.stack([pad_atom, pu, pde, pu, pde], 1)
    # segment layouts of the angle -> bond -> atom sums: row e (short, rank r among its atom's short
    # rows) is the first bond of triplets pair_offsets[i] + r (s_i - 1) + [0, s_i - 1)
    before = np.concatenate([[0], np.cumsum(short.astype(np.int64))])[:e_cap]  # short rows before e
    centre = np.asarray(b.center[:e_cap], np.int64) if len(b.center) else np.zeros(0, np.int64)
    centre = np.concatenate([centre, np.zeros(e_cap - len(centre), np.int64)])
    rank = before - short_offsets[np.clip(centre, 0, n - 1)]
    eto = np.full(e_cap + 1, pair_offsets[-1], np.int64)
    eto[:ec] = pair_offsets[centre[:ec]] + rank[:ec] * np.maximum(s[centre[:ec]] - 1, 0)
    eto = np.minimum(eto, t_cap)
    # the second-bond CSR's permutation: for row e, by first bond, the triplets with e second
    second_perm = np.full(t_cap, -1, np.int64)
    if not overflow:
        t_real = int(pair_offsets[-1])
        line = lg[:t_real]
        key = np.lexsort((line[:, 2], line[:, 4]))  # by second row, then first row
        second_perm[:t_real] = np.arange(t_real)[key]
    bond_rows = np.full(e_cap, -1, np.int64)
    bond_rows[:len(rows)] = rows  # rows are in (atom, rank) order: the builder's rows are sorted by atom
    return {"d2u": d2u.astype(np.int32), "u2d": u2d.astype(np.int32), "invalid_pairs": invalid,
            "short_counts": s, "short_offsets": short_offsets, "short_edge_matrix": sem.astype(np.int32),
            "pair_offsets": pair_offsets, "overflow": overflow, "line_graph": lg.astype(np.int32),
            "edge_triplet_offsets": eto, "bond_rows": bond_rows.astype(np.int32),
            "second_perm": second_perm.astype(np.int32), "center": center.astype(np.int32),
            "neighbor": neighbor.astype(np.int32), "images": images.astype(np.int32)}


def triplet_set(center, neighbor, images, short, n_edges: int) -> set:
    """Brute force: every ordered pair of two distinct short bonds at a common centre, as
    (centre, (neighbour, image) of the first, (neighbour, image) of the second)."""
    by_atom: dict = {}
    for e in range(n_edges):
        if short[e]:
            by_atom.setdefault(int(center[e]), []).append((int(neighbor[e]), *map(int, images[e])))
    out = set()
    for a, bonds in by_atom.items():
        for x in bonds:
            for y in bonds:
                if x != y:
                    out.add((a, x, y))
    return out


def canonical_order_ok(center, neighbor, images, n_atoms: int, max_image: int = 10) -> bool:
    """The reference's canonical key (fixed_capacity_builder.py:1980-1987) is strictly increasing."""
    radix = 2 * max_image + 1
    key = ((center.astype(np.int64) * n_atoms + neighbor) * radix ** 3 + (images[:, 0] + max_image) * radix * radix
           + (images[:, 1] + max_image) * radix + images[:, 2] + max_image)
    return bool(np.all(np.diff(key) > 0))


def reverse(center, neighbor, images, edge_offsets, e_cap: int) -> np.ndarray:
    """Row of (neighbour, centre, -image) for each real row, -1 if not stored."""
    total = int(edge_offsets[-1])
    ec = min(total, e_cap)
    rows = {(int(center[e]), int(neighbor[e]), *map(int, images[e])): e for e in range(ec)}
    out = np.full(e_cap, -1, np.int32)
    for e in range(ec):
        out[e] = rows.get((int(neighbor[e]), int(center[e]), *(-int(v) for v in images[e])), -1)
    return out


def dense_pairs(wrapped, cell, cutoff: float) -> dict:
    """FP64 O(N^2 x images) directed edges {(i, j, nx, ny, nz): distance}
    (tests/test_fixed_capacity_boundary.py:86-102)."""
    pos = np.asarray(wrapped, dtype=np.float64)
    c = np.asarray(cell, dtype=np.float64)
    reach = [int(np.ceil(cutoff / h)) + 1 for h in cell_heights(c)]
    pairs = {}
    for s in np.array(np.meshgrid(*[np.arange(-r, r + 1) for r in reach], indexing="ij")).reshape(3, -1).T:
        v = pos[None, :, :] + (s @ c)[None, None, :] - pos[:, None, :]
        d = np.sqrt((v * v).sum(-1))
        for i, j in zip(*np.nonzero(d < cutoff)):
            if i != j or np.abs(s).sum() > 0:
                pairs[(int(i), int(j), *map(int, s))] = float(d[i, j])
    return pairs


def fixed_capacity_exceeded(edge_count: int, invalid_pairs: bool, e_capacity: int) -> bool:
    """Edges-only rule of fixed_capacity_builder.py:796-814 (fits up to e_capacity inclusive)."""
    return bool(edge_count > e_capacity or invalid_pairs)


def window_fold(state: dict, edges: int, invalid_pairs: bool, overflow: bool, isolated: int, e_cap: int,
                check_isolated: bool) -> dict:
    """_window_flags_kernel (fixed_capacity_builder.py:430-455)."""
    flag = overflow or (check_isolated and isolated > 0)
    return {
        "overflow": state["overflow"] or flag,
        "capacity_overflow": state["capacity_overflow"] or edges > e_cap or invalid_pairs,
        "max_edges": max(state["max_edges"], edges),
        "max_isolated": max(state["max_isolated"], isolated),
    }
