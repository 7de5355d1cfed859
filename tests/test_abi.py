"""The C-ABI library: it exists, loads, and exports every symbol include/fastmd_hip.h declares.
No compute call (CPU suite)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fastmd_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fmd_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_symbols()
    assert "fmd_abi_version" in names and "fmd_nl_build" in names and "fmd_gemm_f32" in names
    assert len(names) >= 15


def test_library_exports_every_declared_symbol():
    from fastmd_amd import _abi

    path = _abi.library_path()
    assert os.path.exists(path), "build the library first (python -m fastmd_amd.csrc.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s+(fmd_[a-z0-9_]+)$", out, flags=re.M))
    missing = [n for n in declared_symbols() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_loader_binds_every_declared_symbol():
    from fastmd_amd import _abi

    lib = _abi.load()
    for name in declared_symbols():
        assert name in _abi.SIGNATURES, f"{name} has no ctypes signature"
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)
    assert lib.fmd_abi_version() == _abi.ABI_VERSION
    assert lib.fmd_error_string(10001).decode().startswith("invalid argument")


def test_gpu_entry_points_refuse_cpu_tensors():
    import torch

    from fastmd_amd.ops.csr_segment_sum import csr_segment_sum

    with pytest.raises(ValueError, match="GPU"):
        csr_segment_sum(torch.ones(3, 2), torch.zeros(3, dtype=torch.long), 1)
