"""The reference's import paths, resolved to this build (the drop-in's import surface).

A caller written against the reference imports, for example,
``from fastmd.ops.triton_gather_cat import aligned_gather_cat3`` or
``from fastmd.execution.gpu_nhc import GPUNoseHooverChainNVT``. After
``install_fastmd_aliases()`` those imports return this build's modules, which keep the
reference's names, signatures and errors. The reference itself keeps such aliases for modules it
moved (fastmd/ops/triton_gather_cat.py:1-6 -> fastmd.models.matris.op.triton_gather_cat, and the
same for triton_csr_segment_sum, triton_weighted_segment_sum, triton_wide_gemm,
triton_threebody_fourier); both the old and the new paths are mapped here.

The aliases are a ``sys.meta_path`` finder: an alias module is imported only when asked for, and
the parent packages (``fastmd``, ``fastmd.ops``, ...) are empty namespace modules. Installing
refuses to shadow a ``fastmd`` package that is already imported (the reference itself).
"""
from __future__ import annotations

import importlib
import importlib.abc
import importlib.machinery
import sys
import types

ALIASES = {
    # operators
    "fastmd.ops.triton_gather_cat": "fastmd_amd.ops.gather_cat",
    "fastmd.models.matris.op.triton_gather_cat": "fastmd_amd.ops.gather_cat",
    "fastmd.ops.triton_csr_segment_sum": "fastmd_amd.ops.csr_segment_sum",
    "fastmd.models.matris.op.triton_csr_segment_sum": "fastmd_amd.ops.csr_segment_sum",
    "fastmd.ops.triton_weighted_segment_sum": "fastmd_amd.ops.segment",
    "fastmd.models.matris.op.triton_weighted_segment_sum": "fastmd_amd.ops.segment",
    "fastmd.engine.kernels.segment": "fastmd_amd.ops.segment",
    "fastmd.ops.triton_wide_gemm": "fastmd_amd.ops.wide_gemm",
    "fastmd.engine.kernels.triton_wide_gemm": "fastmd_amd.ops.wide_gemm",
    "fastmd.models.matris.op.triton_wide_gemm": "fastmd_amd.ops.wide_gemm",
    "fastmd.ops.triton_threebody_fourier": "fastmd_amd.ops.threebody",
    "fastmd.models.matris.op.triton_threebody_fourier": "fastmd_amd.ops.threebody",
    # builder, engine, dispatcher, integrator, runners, driver, outputs
    "fastmd.adapters.protocol": "fastmd_amd.adapters.protocol",
    "fastmd.graph.fixed_capacity_builder": "fastmd_amd.graph.fixed_capacity_builder",
    "fastmd.graph.gpu_graph_builder": "fastmd_amd.graph.gpu_graph_builder",
    "fastmd.graph.neighbor_list_backend": "fastmd_amd.graph.neighbor_list_backend",
    "fastmd.engine.energy_derivative": "fastmd_amd.engine.energy_derivative",
    "fastmd.engine.dispatch": "fastmd_amd.engine.dispatch",
    "fastmd.engine.capacity_policy": "fastmd_amd.engine.capacity_policy",
    "fastmd.engine._graph_capture": "fastmd_amd.execution.graph_capture",
    "fastmd.execution.gpu_integrator": "fastmd_amd.execution.gpu_integrator",
    "fastmd.execution.gpu_nhc": "fastmd_amd.execution.gpu_nhc",
    "fastmd.execution.whole_step_cuda_graph": "fastmd_amd.execution.whole_step_cuda_graph",
    "fastmd.execution.cuda_graph": "fastmd_amd.execution.cuda_graph",
    "fastmd.execution.replica_batch": "fastmd_amd.execution.replica_batch",
    "fastmd.execution.skin_topology": "fastmd_amd.execution.skin_topology",
    "fastmd.execution.system_batch": "fastmd_amd.execution.system_batch",
    "fastmd.interfaces.multi_system_md": "fastmd_amd.interfaces.multi_system_md",
    "fastmd.applications.skin_topology": "fastmd_amd.execution.skin_topology",
    "fastmd.execution.gpu_logging": "fastmd_amd.execution.gpu_logging",
    "fastmd.execution.md_protocol": "fastmd_amd.execution.md_protocol",
    "fastmd.interfaces.gpu_md": "fastmd_amd.interfaces.gpu_md",
    "fastmd._nvtx": "fastmd_amd._roctx",
}

_PACKAGES = frozenset(name.rsplit(".", k)[0] for name in ALIASES for k in range(1, name.count(".") + 1))


class _AliasLoader(importlib.abc.Loader):
    def __init__(self) -> None:
        self._own_specs: dict = {}

    def create_module(self, spec):
        if spec.name in _PACKAGES and spec.name not in ALIASES:
            module = types.ModuleType(spec.name, f"alias package of this build ({spec.name})")
            module.__path__ = []
            return module
        module = importlib.import_module(ALIASES[spec.name])
        self._own_specs[spec.name] = module.__spec__
        return module

    def exec_module(self, module):
        # importlib stamps the alias spec on the module create_module returned; a module of this
        # build gets its own spec back
        own = self._own_specs.pop(module.__spec__.name, None)
        if own is not None:
            module.__spec__ = own


class _AliasFinder(importlib.abc.MetaPathFinder):
    _loader = _AliasLoader()

    def find_spec(self, fullname, path=None, target=None):
        if fullname not in ALIASES and fullname not in _PACKAGES:
            return None
        return importlib.machinery.ModuleSpec(fullname, self._loader, is_package=fullname in _PACKAGES)


_FINDER = _AliasFinder()


def install_fastmd_aliases() -> None:
    """Make the reference's ``fastmd.*`` import paths (``ALIASES``) resolve to this build."""
    existing = sys.modules.get("fastmd")
    if existing is not None and getattr(existing, "__path__", None) != []:
        raise RuntimeError("a fastmd package is already imported; the aliases would shadow it")
    if _FINDER not in sys.meta_path:
        sys.meta_path.insert(0, _FINDER)


def uninstall_fastmd_aliases() -> None:
    """Remove the finder and every ``fastmd`` alias module from ``sys.modules``."""
    if _FINDER in sys.meta_path:
        sys.meta_path.remove(_FINDER)
    for name in [n for n in sys.modules if n == "fastmd" or n.startswith("fastmd.")]:
        del sys.modules[name]
