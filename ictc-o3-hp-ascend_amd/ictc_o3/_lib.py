"""ctypes binding of libictc_hip.so (the C ABI declared in include/ictc_hip.h).

torch is imported before the library is opened: torch-ROCm ships its own HIP
runtime with the same SONAME (libamdhip64.so.7), so the library's dependency then
resolves to the runtime torch already loaded and both share streams and memory.
There is no fallback: if the library is missing every operator raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede CDLL, see module docstring)

MAX_PATHS = 128
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libictc_hip.so")
ABI_VERSION = 21


class TpDesc(ctypes.Structure):
    """Mirror of ``ictc_tp_desc``."""
    _fields_ = [
        ("channels", ctypes.c_int32),
        ("input_lmax", ctypes.c_int32),
        ("edge_lmax", ctypes.c_int32),
        ("output_lmax", ctypes.c_int32),
        ("num_paths", ctypes.c_int32),
        ("out_components", ctypes.c_int32),
        ("gate_index", ctypes.c_int32 * MAX_PATHS),
        ("out_offset", ctypes.c_int32 * MAX_PATHS),
        ("scale", ctypes.c_float * MAX_PATHS),
    ]


class DegreeLinearDesc(ctypes.Structure):
    """Mirror of ``ictc_degree_linear_desc``."""
    _fields_ = [
        ("lmax", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("out_channels", ctypes.c_int32),
        ("counts", ctypes.c_int32 * 8),
    ]


class CellGrid(ctypes.Structure):
    """Mirror of ``ictc_cell_grid``."""
    _fields_ = [
        ("cell", ctypes.c_double * 9),
        ("cutoff_sq", ctypes.c_double),
        ("bins", ctypes.c_int32 * 3),
        ("reach", ctypes.c_int32 * 3),
        ("periodic", ctypes.c_int32 * 3),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SIGNATURES = {
    "ictc_hip_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "ictc_hip_abi_version": (ctypes.c_int, []),
    "ictc_hip_tp_slot_count": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "ictc_hip_tp_forward": (ctypes.c_int, [ctypes.POINTER(TpDesc), _P, _P, _P, _P, _I64, _P]),
    "ictc_hip_tp_backward": (ctypes.c_int, [ctypes.POINTER(TpDesc), _P, _P, _P, _P, _P, _P, _P,
                                            _I64, _P]),
    "ictc_hip_direction_harmonics": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _P, _P, _P, _P, _P,
                                                    _I64, _P]),
    "ictc_hip_message_chunks": (ctypes.c_int, [ctypes.c_int]),
    "ictc_hip_sc_weight_columns": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "ictc_hip_sc_forward": (ctypes.c_int, [ctypes.c_int] * 4 + [_P, _P, _P, ctypes.c_int, _P, _I64, _P]),
    "ictc_hip_sc_backward": (ctypes.c_int, [ctypes.c_int] * 4 + [_P, _P, _P, ctypes.c_int, _P, _P, _I64,
                                                                   _P]),
    "ictc_hip_sc_weight_features": (ctypes.c_int, [ctypes.c_int] * 4 + [_P, _P, ctypes.c_int, _P, _P, _I64,
                                                                          _P]),
    "ictc_hip_sc_jvp": (ctypes.c_int, [ctypes.c_int] * 4 + [_P, _P, _P, ctypes.c_int, _P, _P, _I64, _P]),
    "ictc_hip_sc_hvp": (ctypes.c_int, [ctypes.c_int] * 4 + [_P, _P, _P, ctypes.c_int, _P, _P, _P, _I64, _P]),
    "ictc_hip_sc_weight_features_jvp": (ctypes.c_int, [ctypes.c_int] * 4 + [_P, _P, ctypes.c_int, _P, _P, _P,
                                                                              _I64, _P]),
    "ictc_hip_message_bond_width": (ctypes.c_int, [ctypes.POINTER(TpDesc)]),
    "ictc_hip_message_bonds": (ctypes.c_int, [ctypes.POINTER(TpDesc), _P, _P, _I64, _P]),
    "ictc_hip_message_forward": (ctypes.c_int, [ctypes.POINTER(TpDesc), _P, _P, _P, _P, _P, _P, _P,
                                                _I64, _I64, _I64, _P]),
    "ictc_hip_message_edge_grad": (ctypes.c_int, [ctypes.POINTER(TpDesc), _P, _P, _P, _P, _P, _P, _P,
                                                  _P, _P, _P, _I64, _I64, _I64, ctypes.c_int, _P]),
    "ictc_hip_message_static_prepare": (ctypes.c_int, []),
    "ictc_hip_message_edge_grad_static": (ctypes.c_int, [ctypes.POINTER(TpDesc), _P, _P, _P, _P, _P, _P, _P,
                                                         _P, _P, _P, _I64, _I64, _I64, _P]),
    "ictc_hip_message_node_grad": (ctypes.c_int, [ctypes.POINTER(TpDesc), _P, _P, _P, _P, _I64, _I64, _P]),
    "ictc_hip_message_forward_tangent": (ctypes.c_int, [ctypes.POINTER(TpDesc)] + [_P] * 10 + [_I64, _I64, _I64,
                                                                                          _P]),
    "ictc_hip_message_edge_grad_tangent": (ctypes.c_int, [ctypes.POINTER(TpDesc)] + [_P] * 13 + [_I64, _I64,
                                                                                            _I64, _P]),
    "ictc_hip_edge_vector_grad": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "ictc_hip_degree_linear_forward": (ctypes.c_int, [ctypes.POINTER(DegreeLinearDesc), _P, _P, ctypes.c_float, _P,
                                                      _I64, _P]),
    "ictc_hip_degree_linear_input_grad": (ctypes.c_int, [ctypes.POINTER(DegreeLinearDesc), _P, _P, ctypes.c_float,
                                                         _P, _I64, _P]),
    "ictc_hip_degree_linear_mul_ir": (ctypes.c_int, [ctypes.POINTER(DegreeLinearDesc), _P, _P, ctypes.c_float, _P,
                                                     _I64, _P]),
    "ictc_hip_degree_linear_mul_ir_transposed": (ctypes.c_int, [ctypes.POINTER(DegreeLinearDesc), _P, _P,
                                                                ctypes.c_float, _P, _I64, _P]),
    "ictc_hip_degree_linear_weight_grad_workspace": (_I64, [ctypes.POINTER(DegreeLinearDesc), ctypes.c_int, _I64]),
    "ictc_hip_degree_linear_weight_grad": (ctypes.c_int, [ctypes.POINTER(DegreeLinearDesc), ctypes.c_int, _P, _P,
                                                          ctypes.c_float, _P, _I64, _P, _I64, _P]),
    "ictc_hip_silu_second": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _P]),
    "ictc_hip_readout": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _P, ctypes.c_int,
                                        ctypes.c_int, _I64, _P]),
    "ictc_hip_species_linear": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, ctypes.c_int, ctypes.c_int, _I64, _P]),
    "ictc_hip_edge_embedding": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, _P, _P, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_float, _I64, _P]),
    "ictc_hip_radial_mlp_workspace": (_I64, [_I64]),
    "ictc_hip_radial_mlp": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _P, _P, _P, _I64,
                                           _P, _P, _P, ctypes.c_int, _I64, _P]),
    "ictc_hip_sgemm": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _I64, _I64, _I64, ctypes.c_float, _P, _I64, _P,
                                      _I64, ctypes.c_float, _P, _I64, _P]),
    "ictc_hip_radius_graph_count": (ctypes.c_int, [ctypes.POINTER(CellGrid), _P, _P, _P, _P, _I64, _P, _P]),
    "ictc_hip_radius_graph_fill": (ctypes.c_int, [ctypes.POINTER(CellGrid), _P, _P, _P, _P, _I64, _P, _P, _P,
                                                  _P]),
    "ictc_hip_radius_graph_row_capacity": (_I64, []),
    "ictc_hip_radius_graph_fill_sorted": (ctypes.c_int, [ctypes.POINTER(CellGrid), _P, _P, _P, _P, _I64, _P, _P, _P,
                                                         _P, _P, _P]),
}

_lock = threading.Lock()
_lib = None


def exported_symbols():
    """Names of every entry point the binding expects (the header's declarations)."""
    return tuple(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """Open (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.isfile(LIB_PATH):
                raise RuntimeError(
                    f"libictc_hip.so not found at {LIB_PATH}; build it with "
                    "`python ictc-o3-hp-ascend_amd/csrc/build.py` (no CPU fallback exists)")
            handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = res, args
            if handle.ictc_hip_abi_version() != ABI_VERSION:
                raise RuntimeError("libictc_hip.so ABI version mismatch; rebuild the library")
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().ictc_hip_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """Handle of torch's current stream on device (the raw query: ~0.06 us against ~1.8 us for
    building a torch.cuda.Stream object, on a path issued a hundred times per MACE step)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream
