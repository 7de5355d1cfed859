"""ctypes binding of ``libfastmd_hip.so`` (the C ABI declared in ``include/fastmd_hip.h``).

The library is loaded after ``torch`` so that it binds the HIP runtime torch already loaded
(one runtime per process: streams and device pointers are shared). There is no fallback: if
the library is missing, every GPU entry point raises ``RuntimeError`` naming the build step.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime the library binds)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libfastmd_hip.so")
ABI_VERSION = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_u8 = ctypes.c_uint8

# name -> (restype, argtypes); mirrors include/fastmd_hip.h
SIGNATURES: dict[str, tuple] = {
    "fmd_abi_version": (ctypes.c_int, []),
    "fmd_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "fmd_nl_candidates": (ctypes.c_int, [_p, _p, _p, _i64, _f32, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _i64,
                                         _i64, _p]),
    "fmd_nl_wrap": (ctypes.c_int, [_p, _i32, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p]),
    "fmd_nl_build_work_size": (_i64, [_i64]),
    "fmd_nl_build": (ctypes.c_int, [_p, _i32, _p, _p, _i64, _p, _p, _p, _i32, _p, _p, _p, _f32, _f32, _i32,
                                    _i32, _i32, _i32, _i32, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                    _p, _p, _p, _p, _p, _f32, _p, _p, _p, _p, _p, _p, _p, _i32, _p]),
    "fmd_nl_build_noalloc": (ctypes.c_int, [_p, _i32, _p, _p, _i64, _p, _p, _p, _i32, _p, _p, _p, _f32, _f32, _i32,
                                            _i32, _i32, _i32, _i32, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                            _p, _p, _p, _p, _p, _f32, _p, _p]),
    "fmd_nl_line_graph_work_size": (_i64, [_i64, _i64]),
    "fmd_nl_line_graph": (ctypes.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _p,
                                         _p, _p, _p, _p, _p, _p, _p, _p, _i32, _p]),
    "fmd_threebody_fourier_f32": (ctypes.c_int, [_p, _i64, _p, _p, _i64, _p, _i32, _f32, _p, _p]),
    "fmd_threebody_fourier_bwd_rows_f32": (ctypes.c_int, [_p, _p, _i64, _p, _p, _i64, _p, _i32, _f32, _p, _p]),
    "fmd_threebody_fourier_line_f32": (ctypes.c_int, [_p, _i64, _p, _p, _p, _i32, _p, _p, _i64, _i64, _p, _i32, _f32,
                                                      _p, _p]),
    "fmd_threebody_fourier_line_bwd_f32": (ctypes.c_int, [_p, _p, _i64, _p, _p, _p, _i32, _p, _i64, _i64, _p, _i32,
                                                          _f32, _p, _i64, _i32, _p]),
    "fmd_tb_bond_envelope_f32": (ctypes.c_int, [_p, _p, _p, _i64, _f32, _p]),
    "fmd_tb_gated_sum_f32": (ctypes.c_int, [_p, _i64, _i64, _i32, _p, _i64, _p, _p, _i64, _p, _i64, _f32, _p, _i64,
                                            _i32, _p]),
    "fmd_tb_gated_sum_bwd_f32": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _i32, _p, _i64, _p, _p, _i64, _p, _i64,
                                                _f32, _p, _i64, _p, _i64, _p, _i64, _i32, _p]),
    "fmd_tb_bond_sum_f32": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _p, _p, _i64, _i64, _f32, _p, _i64, _p]),
    "fmd_tb_triplet_bwd_f32": (ctypes.c_int, [_p, _i64, _p, _i64, _i32, _p, _p, _p, _i64, _i64, _f32, _p, _i64, _p,
                                              _p]),
    "fmd_tb_bond_reduce_f32": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _p, _i32,
                                              _p]),
    "fmd_tb_readout_f32": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _i64, _p, _p]),
    "fmd_tb_readout_bwd_f32": (ctypes.c_int, [_p, _f32, _p, _i32, _i64, _p, _i64, _p]),
    "fmd_tb_geometry_bwd_f32": (ctypes.c_int, [_p, _p, _i32, _p, _i64, _p, _i64, _p, _p, _p, _p, _i64, _p, _p]),
    "fmd_nl_reverse": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i64, _p, _p]),
    "fmd_nl_pad_rows": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _p]),
    "fmd_nl_window_flags": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p]),
    "fmd_gather_cat_f32": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _i64, _p, _i64, _p]),
    "fmd_segsum_csr_f32": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32,
                                          _p, _i64, _p]),
    "fmd_segsum_csr_t_f32": (ctypes.c_int, [_p, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _p, _p,
                                            _p]),
    "fmd_gemm_f32": (ctypes.c_int, [_p, _i64, _p, _i64, _i32, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "fmd_gemm_group_f32": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _i32,
                                          _p]),
    "fmd_gemm_group_ks_f32": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32,
                                             _p]),
    "fmd_gemm_group_x3_planes_f32": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                                    _i32, _p]),
    "fmd_gemm_group_x3_planes_rows_f32": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                                         _p, _p, _p, _p, _i32, _p]),
    "fmd_split3_f32": (ctypes.c_int, [_p, _i64, _i64, _i32, _p, _p]),
    "fmd_gemm_x3_planes_f32": (ctypes.c_int, [_i32, _i32, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _p, _p, _i64,
                                              _i64, _p, _p, _i64, _i64, _i32, _i32, _p]),
    "fmd_gemm_splitk_x3_planes_f32": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _p, _i64, _p, _p, _i64, _i64, _i64,
                                                      _i64, _i32, _i32, _p, _p]),
    "fmd_gemm_splitk_f32": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _p, _i64, _i32, _p, _p, _i64, _i64, _i64, _i64,
                                           _i32, _i32, _p, _p]),
    "fmd_gemm_gather_f32": (ctypes.c_int, [_i32, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _p, _p, _i64,
                                           _i64, _i32, _i32, _p]),
    "fmd_gemm_bf16": (ctypes.c_int, [_p, _i64, _p, _i64, _i32, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "fmd_nhc_pre_force": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _p, _p]),
    "fmd_nhc_post_force": (ctypes.c_int, [_p, _p, _i32, _p, _p, _p, _p, _p, _p, _i32, _p, _i64, _i32, _i32,
                                          _i32, _p, _p]),
    "fmd_nhc_post_pre": (ctypes.c_int, [_p, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _i32, _p, _i64, _i32, _i32, _i32,
                                        _p, _p]),
    "fmd_nhc_work_size": (_i64, [_i64]),
    "fmd_sum_f64": (ctypes.c_int, [_p, _i32, _i64, _p, _p]),
    "fmd_edge_geometry_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _i64, _f32, _i32, _p, _p, _p, _p]),
    "fmd_edge_geometry_bwd_f32": (ctypes.c_int, [_p, _p, _i32, _p, _i64, _p, _i64, _p, _p, _i64, _p, _p]),
    "fmd_mace_message_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _p, _i32, _p, _p, _f32, _p, _p, _i32,
                                            _p, _p, _i32, _i32, _p]),
    "fmd_mace_message_bwd_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _i32, _p, _p, _p, _p, _f32,
                                                _p, _p, _p, _p, _i32, _p, _p, _i32, _p, _i32, _p, _i32, _p, _i32, _p]),
    "fmd_mace_node_fwd_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p, _p, _p, _p, _p,
                                             _p, _p]),
    "fmd_mace_node_bwd_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p, _p, _p, _i32,
                                             _p, _p, _p, _p, _p]),
    "fmd_mace_mix_symcon_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p, _p, _p, _p, _p]),
    "fmd_mace_mix_symcon_bwd_f32": (ctypes.c_int, [_p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p, _p,
                                                   _p]),
    "fmd_mace_symcon_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _i64, _i32, _p, _p, _p]),
    "fmd_mace_symcon_bwd_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p, _p, _p]),
    "fmd_mace_energy_f32": (ctypes.c_int, [_p, _p, _p, _p, _i32, _i32, _p, _p, _f32, _f32, _i64, _p, _p]),
    "fmd_mace_energy_bwd_f32": (ctypes.c_int, [_p, _p, _p, _p, _i32, _i32, _f32, _i64, _p, _p, _p]),
    "fmd_mace_energy_grad_f32": (ctypes.c_int, [_p, _p, _p, _p, _i32, _i32, _p, _p, _f32, _f32, _i64, _p, _p, _p,
                                                _p, _p, _p]),
    "fmd_embed_f32": (ctypes.c_int, [_p, _p, _i64, _i32, _p, _p]),
    "fmd_embed_rows_f32": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _p]),
    "fmd_edge_geometry_embed_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _i64, _f32, _i32, _p, _p, _p, _p, _i64,
                                                   _i32, _p, _p, _p, _p]),
    "fmd_morse_f32": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _f32, _f32, _f32, _f32, _f32, _p, _p, _p]),
    "fmd_morse_bwd_f32": (ctypes.c_int, [_p, _p, _p, _p, _p, _i64, _p, _p]),
    "fmd_edge_virial_work_size": (_i64, []),
    "fmd_nl_overflow_rows": (ctypes.c_int, [_p, _i64, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p]),
    "fmd_nl_pad_override": (ctypes.c_int, [_p, _i64, _f32, _f32, _f32, _p, _p]),
    "fmd_edge_stress_f32": (ctypes.c_int, [_p, _p, _p, _i64, _p, _p, _p, _p]),
}

_lock = threading.Lock()
_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """The loaded library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m fastmd_amd.csrc.build` "
                "(or __graft_entry__.build()); there is no CPU fallback for the MI355X kernels")
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.fmd_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int, name: str) -> None:
    if status != 0:
        message = load().fmd_error_string(int(status)).decode(errors="replace")
        raise RuntimeError(f"{name} failed with status {status}: {message}")


def call(name: str, *args) -> None:
    """Call ``name`` and raise ``RuntimeError`` on a nonzero status."""
    check(getattr(load(), name)(*args), name)


def ptr(tensor) -> int | None:
    """Device address of a tensor (None for None)."""
    if tensor is None:
        return None
    return tensor.data_ptr()


def stream_handle(device=None) -> int:
    """torch's current HIP stream (the stream every entry point launches on)."""
    return torch.cuda.current_stream(device).cuda_stream


def array(ctype, values):
    """A host C array (for the pointer-array arguments of the multi-part entry points)."""
    values = list(values)
    return (ctype * max(1, len(values)))(*values)


def ptr_array(values):
    return array(ctypes.c_void_p, [0 if v is None else v for v in values])
