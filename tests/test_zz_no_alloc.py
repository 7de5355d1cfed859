"""fmd_nl_build_noalloc, the allocation-free neighbour-list build (its per-block partials in a
static device array instead of a caller's work buffer), against fmd_nl_build on the same
inputs: every output bitwise equal, on calls in a row with shrinking systems (2 560 atoms, then
1 080 on the multi-block path, then 135 on the single-workgroup path), and FMD_ETOOLARGE above
the array's atom limit with nothing launched."""
import numpy as np
import pytest

from fastmd_amd import systems
from fastmd_amd.adapters.protocol import PaddingRule

# the builder's output buffers of one build (persistent tensors the C ABI writes)
OUTPUTS = ("frac_coords", "wrap_delta", "positions", "edge_counts", "edge_offsets", "center", "neighbor", "images",
           "distances", "_max_displacement", "_candidate_valid", "_overflow", "_isolated_atom_count")
MAX_ATOMS = 1 << 20  # FMD_NL_BUILD_NOALLOC_MAX_ATOMS
ETOOLARGE = 10003


def _outputs(builder):
    out = {name: getattr(builder, name) for name in OUTPUTS}
    out["edge_index"] = builder.batch.edge_index
    out["edge_image"] = builder.batch.edge_image
    return out


def _noalloc_args(builder, positions, out, n_atoms=None):
    from fastmd_amd import _abi

    image = builder._pad_image
    return (positions.data_ptr(), 1, builder.inv_cell.data_ptr(), builder.cell.data_ptr(),
            builder.n_real if n_atoms is None else n_atoms, builder.neighbor_matrix.data_ptr(),
            builder.neighbor_shifts.data_ptr(), builder.num_neighbors.data_ptr(), builder.buffer_max,
            builder.reference_positions.data_ptr(), builder.reference_wraps.data_ptr(),
            builder._candidate_capacity_valid.data_ptr(), builder._rc2, builder._skin_limit,
            1 if builder.minimum_image else 0, image[0], image[1], image[2], builder.n_dummy, None, None,
            builder.e_capacity, out["frac_coords"].data_ptr(), out["wrap_delta"].data_ptr(),
            out["positions"].data_ptr(), out["edge_counts"].data_ptr(), out["edge_offsets"].data_ptr(),
            out["center"].data_ptr(), out["neighbor"].data_ptr(), out["images"].data_ptr(),
            out["distances"].data_ptr(), out["edge_index"].data_ptr(), out["edge_image"].data_ptr(),
            out["_max_displacement"].data_ptr(), out["_candidate_valid"].data_ptr(), out["_overflow"].data_ptr(),
            out["_isolated_atom_count"].data_ptr(), builder._line2, _abi.ptr(builder.short_flags),
            _abi.stream_handle(builder.device))


@pytest.mark.gpu
def test_noalloc_build_equals_the_build_with_a_work_buffer(device):
    import torch

    from fastmd_amd import _abi
    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    for k in (8, 6, 3):
        s = systems.perovskite(k)
        n = s.n_atoms
        print(f"[noalloc] {n} atoms", flush=True)
        builder = FixedCapacityGraphBuilder(cell=torch.tensor(s.cell, dtype=torch.float32),
                                            atomic_numbers=torch.ones(n), u_capacity=9 * n + 64, t_capacity=0,
                                            line_graph_cutoff=None, atom_graph_cutoff=6.0, candidate_cutoff=8.0,
                                            padding=PaddingRule("far_self_loops"), device=device)
        pos = torch.tensor(s.positions, dtype=torch.float64, device=device)
        builder.build(pos, rebuild_candidates=True)
        # a step later: atoms moved (wraps change near the cell faces), the candidates reused
        moved = s.positions + np.random.default_rng(k).normal(0, 0.08, s.positions.shape)
        moved = torch.tensor(moved, dtype=torch.float64, device=device)
        before = {name: t.clone() for name, t in _outputs(builder).items()}
        builder.build(moved, rebuild_candidates=False)
        expected = {name: t.clone() for name, t in _outputs(builder).items()}
        got = {name: t.clone() for name, t in before.items()}  # the same prior contents
        _abi.call("fmd_nl_build_noalloc", *_noalloc_args(builder, moved, got))
        torch.cuda.synchronize()
        for name in expected:
            assert torch.equal(got[name], expected[name]), (n, name)
        e = int(expected["edge_offsets"][-1])
        assert e > 10 * n and int(expected["_overflow"][0]) == 0
    # beyond the static array: a clear error, nothing launched (the sizes are checked first)
    status = _abi.load().fmd_nl_build_noalloc(*_noalloc_args(builder, moved, got, n_atoms=MAX_ATOMS + 1))
    assert status == ETOOLARGE
    assert "allocation-free" in _abi.load().fmd_error_string(status).decode()
