"""The reference's import paths (``fastmd.*``) resolve to this build after
``install_fastmd_aliases()``: every path imports and carries the reference's names (CPU); the
operator functions imported by their reference paths run on the HIP kernels and match PyTorch
(GPU)."""
import importlib

import numpy as np
import pytest

from fastmd_amd.aliases import ALIASES, install_fastmd_aliases, uninstall_fastmd_aliases
from fastmd_amd.adapters.protocol import PaddingRule

REFERENCE_NAMES = {
    "fastmd.ops.triton_gather_cat": ("aligned_gather_cat3", "aligned_gather_cat4"),
    "fastmd.ops.triton_csr_segment_sum": ("csr_segment_sum",),
    "fastmd.ops.triton_weighted_segment_sum": ("weighted_segment_sum",),
    "fastmd.engine.kernels.segment": ("aggregate", "segment_count"),
    "fastmd.ops.triton_wide_gemm": ("linear", "linear_into", "matmul"),
    "fastmd.engine.kernels.triton_wide_gemm": ("linear", "linear_into", "matmul"),
    "fastmd.ops.triton_threebody_fourier": ("threebody_fourier_basis",),
    "fastmd.adapters.protocol": ("GraphBatch", "PaddingRule", "CapacityStep", "CaptureContract", "ModelAdapter",
                                 "EnergyTap"),
    "fastmd.graph.fixed_capacity_builder": ("FixedCapacityGraphBuilder", "FixedCapacityGraphStatus",
                                            "fixed_capacity_exceeded", "self_loop_padding"),
    "fastmd.graph.gpu_graph_builder": ("TensorGraphBuilder",),
    "fastmd.graph.neighbor_list_backend": ("estimate_max_neighbors", "NeighborOverflowError"),
    "fastmd.engine.energy_derivative": ("EnergyDerivative",),
    "fastmd.engine.capacity_policy": ("tier", "held_demand", "JointCapacityPolicy"),
    "fastmd.engine._graph_capture": ("capture_graph", "CAPTURE_ERROR_MODE"),
    "fastmd.execution.gpu_integrator": ("StatefulIntegrator",),
    "fastmd.execution.gpu_nhc": ("GPUNoseHooverChainNVT", "nhc_constants", "maxwell_boltzmann_momenta", "NHCState"),
    "fastmd.execution.whole_step_cuda_graph": ("WholeStepGraphRunner", "FixedCapacityOverflow"),
    "fastmd.execution.cuda_graph": ("BucketedGraphRunner",),
    "fastmd.execution.replica_batch": ("ReplicaNoseHooverChainNVT",),
    "fastmd.execution.skin_topology": ("SkinTopologyRunner", "SkinTopologyUnavailable", "PROACTIVE_REFRESH_FRACTION"),
    "fastmd.execution.system_batch": ("SlotLayout", "SlotUnionGraphBuilder", "SystemNoseHooverChainNVT"),
    "fastmd.interfaces.multi_system_md": ("MultiSystemMolecularDynamics",),
    "fastmd.execution.gpu_logging": ("AsyncGPUMDLogger",),
    "fastmd.execution.md_protocol": ("MDOutputs", "ExtxyzTrajectory", "RestartData", "read_restart", "write_restart",
                                     "resume_mismatch"),
    "fastmd.interfaces.gpu_md": ("GPUResidentMolecularDynamics",),
    "fastmd._nvtx": ("nvtx_range", "nvtx_ranged"),
}


@pytest.fixture
def aliases():
    install_fastmd_aliases()
    try:
        yield
    finally:
        uninstall_fastmd_aliases()


def test_every_reference_path_resolves_with_its_names(aliases):
    assert set(REFERENCE_NAMES) <= set(ALIASES)
    for path, target in ALIASES.items():
        module = importlib.import_module(path)
        assert module is importlib.import_module(target), path
        assert module.__spec__.name == target  # this build's module keeps its own spec
        for name in REFERENCE_NAMES.get(path, ()):
            assert hasattr(module, name), (path, name)
    from fastmd.engine._graph_capture import CAPTURE_ERROR_MODE
    from fastmd._nvtx import nvtx_range

    assert CAPTURE_ERROR_MODE == "thread_local"
    with nvtx_range("alias test"):  # a no-op or a roctx range, never an error
        pass


def test_aliases_refuse_to_shadow_an_imported_fastmd():
    import sys
    import types

    sys.modules["fastmd"] = types.ModuleType("fastmd")  # stands for the reference's own package
    try:
        with pytest.raises(RuntimeError, match="already imported"):
            install_fastmd_aliases()
    finally:
        del sys.modules["fastmd"]
    uninstall_fastmd_aliases()


@pytest.mark.gpu
def test_reference_paths_run_the_hip_operators(device, aliases):
    import torch

    from fastmd.engine.kernels.triton_wide_gemm import linear
    from fastmd.ops.triton_csr_segment_sum import csr_segment_sum
    from fastmd.ops.triton_gather_cat import aligned_gather_cat3
    from fastmd.ops.triton_weighted_segment_sum import weighted_segment_sum

    g = torch.Generator().manual_seed(3)
    n, e, f = 40, 300, 64
    x = torch.randn(n, f, generator=g)
    aligned = torch.randn(e, 8, generator=g)
    ia = torch.randint(0, n, (e,), generator=g)
    ib = torch.sort(torch.randint(0, n, (e,), generator=g)).values
    out = aligned_gather_cat3(aligned.to(device), x.to(device), ia.to(device), ib.to(device))
    assert torch.equal(out.cpu(), torch.cat([aligned, x[ia], x[ib]], 1))
    v = torch.randn(e, f, generator=g)
    ref = torch.zeros(n, f, dtype=torch.float64).index_add_(0, ib, v.double())
    got = csr_segment_sum(v.to(device), ib.to(device), n)
    assert float((got.cpu().double() - ref).abs().max() / ref.abs().max()) < 1e-5
    w = torch.randn(e, f, generator=g)
    refw = torch.zeros(n, f, dtype=torch.float64).index_add_(0, ib, (w * v).double())
    gotw = weighted_segment_sum(w.to(device), v.to(device), ib.to(device), n)
    assert float((gotw.cpu().double() - refw).abs().max() / refw.abs().max()) < 1e-5
    a, wt = torch.randn(e, 136, generator=g), torch.randn(96, 136, generator=g)
    y = linear(a.to(device), wt.to(device))
    ref_y = a.double() @ wt.double().T
    assert float((y.cpu().double() - ref_y).abs().max() / ref_y.abs().max()) < 1e-5


@pytest.mark.gpu
def test_reference_paths_run_the_builder_and_integrator(device, aliases):
    import torch

    from fastmd.execution.gpu_nhc import GPUNoseHooverChainNVT, maxwell_boltzmann_momenta
    from fastmd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder
    from fastmd_amd import systems

    s = systems.perovskite(3)
    builder = FixedCapacityGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers),
                                        u_capacity=1088, t_capacity=0, line_graph_cutoff=None, atom_graph_cutoff=6.0,
                                        candidate_cutoff=8.0, padding=PaddingRule("far_self_loops"), device=device)
    _, status = builder.build(torch.tensor(s.positions, device=device))
    assert not bool(status.overflow.item()) and int(status.edge_count.item()) == 2054
    from fastmd_amd import units

    nhc = GPUNoseHooverChainNVT(s.masses, s.positions, maxwell_boltzmann_momenta(s.masses, 500.0, 0),
                                temperature_K=500.0, timestep=0.25 * units.fs, tdamp=25.0 * units.fs,
                                device=device)
    q = nhc.step_pre_force()
    nhc.step_post_force(torch.zeros_like(q, dtype=torch.float32))
    assert np.isfinite(float(nhc.conserved_energy()))
