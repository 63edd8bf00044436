"""ctypes binding of libictc_mi355x.so (the C ABI in include/ictc_mi355x.h).

The library is built in-tree by ``csrc/build.py``.  There is no fallback:
if the library is missing, or the tensors are not on a ROCm device, every
entry point raises.  Launches go on torch's current HIP stream of the
operand's device, so they order correctly with surrounding torch work.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libictc_mi355x.so")
_lock = threading.Lock()
_lib = None

_i = ctypes.c_int
_i64 = ctypes.c_int64
_p = ctypes.c_void_p

_SIGNATURES = {
    "ictc_version": (_i, []),
    "ictc_last_error": (ctypes.c_char_p, []),
    "ictc_tp_shape": (_i, [_i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "ictc_tp_fwd": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _i64, _p, _p]),
    "ictc_tp_workspace_bytes": (_i64, [_i, _i, _i64]),
    "ictc_tp_bwd": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _i64, _p]),
    "ictc_tp_second": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _i64, _p]),
    "ictc_msg_second": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p,
                             _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "ictc_csr_workspace_bytes": (_i64, [_i64, _i64]),
    "ictc_csr_build": (_i, [_p, _i64, _i64, _p, _p, _p, _i64, _p]),
    "ictc_morton_workspace_bytes": (_i64, [_i64]),
    "ictc_morton_order": (_i, [_p, _i64, ctypes.c_float, _p, _p, _i64, _p]),
    "ictc_receiver_rows_workspace_bytes": (_i64, [_i64]),
    "ictc_receiver_rows": (_i, [_p, _i64, _p, _p, _p, _i64, _p]),
    "ictc_msg_fwd": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p]),
    "ictc_msg_bwd": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p,
                          _p, _p, _p, _p, _p, _p, _i64, _p]),
    "ictc_msg_bwd_accumulate": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p,
                                     _p, _p, _p, _p, _p, _p, _i64, _p]),
    "ictc_msg_bwd_tangent_workspace_bytes": (_i64, [_i, _i, _i64]),
    "ictc_msg_bwd_tangent": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p,
                                  _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p]),
    "ictc_fused_supported": (_i, [_i, _i, _i, _i]),
    "ictc_fused_weight_bytes": (_i64, [_i, _i]),
    "ictc_fused_weight_split": (_i, [_p, _p, _i, _i, _p, _i64, _p]),
    "ictc_species_message_workspace_bytes": (_i64, [_i, _i, _i, _i64]),
    "ictc_species_message_fwd": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p,
                                      _p, _i64, _p]),
    "ictc_species_message_bwd": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p,
                                      _p, _p, _p, _p, _i64, _p]),
    "ictc_msg_fused_fwd": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p]),
    "ictc_msg_fused_bwd_tangent": (_i, [_i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p,
                                        _p, _p, _p, _p, _p, _p, _p, _p]),
    "ictc_edge_pairs_workspace_bytes": (_i64, [_i64]),
    "ictc_edge_pairs": (_i, [_p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "ictc_edge_pairs_src_csr": (_i, [_p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "ictc_sh_fwd": (_i, [_p, _i64, _i, _p, _p]),
    "ictc_sh_bwd": (_i, [_p, _p, _i64, _i, _p, _p]),
    "ictc_sh_jvp": (_i, [_p, _p, _i64, _i, _p, _p]),
    "ictc_sh_hvp": (_i, [_p, _p, _p, _i64, _i, _p, _p]),
    "ictc_silu": (_i, [_i, _p, _p, _p, ctypes.c_float, _i64, _p, _p]),
    "ictc_radial": (_i, [_i, _p, _p, _p, _i64, _i, ctypes.c_float, _i, _p, _p]),
    "ictc_packed_linear": (_i, [_i, _i, _i, _p, _i64, _p, _p, _p, _i64, _p, _p, _p, _p, _i64, _p]),
    "ictc_neighbors_workspace_bytes": (_i64, [_i64, _p]),
    "ictc_neighbors_count": (_i, [_p, _i64, _p, ctypes.c_double, _p, _p, _i64, _p, _p]),
    "ictc_neighbors_fill": (_i, [_p, _i64, _p, ctypes.c_double, _p, _p, _i64, _p, _p, _p, _p]),
    "ictc_neighbors_fill_capacity": (_i, [_p, _i64, _p, ctypes.c_double, _p, _p, _i64, _p, _p, _p, _i64, _p]),
    "ictc_gate_gemm_fwd": (_i, [_p, _i64, _i, _p, _i, _p, _p]),
    "ictc_radial_gates_workspace_bytes": (_i64, [_i]),
    "ictc_radial_gates_fwd": (_i, [_p, _i64, _i, _i, ctypes.c_float, _i, _p, _p, _p, _p, _i, ctypes.c_float, _p, _p,
                                   _i64, _p]),
    "ictc_radial_gates_tangent_fwd": (_i, [_p, _i64, _i, _i, ctypes.c_float, _i, _p, _p, _p, _p, _i,
                                           ctypes.c_float, _p, _p, _p, _i64, _p]),
    "ictc_radial_gates_tangent_fwd_noalloc": (_i, [_p, _i64, _i, _i, ctypes.c_float, _i, _p, _p, _p, _p, _i,
                                                   ctypes.c_float, _p, _p, _p]),
    "ictc_gate_gemm_bwd": (_i, [_p, _i64, _i, _p, _i, _p, _p]),
    "ictc_gate_gemm_bwd_strided": (_i, [_p, _i64, _i64, _i, _p, _i, _p, _i, _p]),
    "ictc_gemm_tn_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "ictc_gemm_nt": (_i, [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i, _p]),
    "ictc_graph_sum": (_i, [_p, _p, _i64, _i64, _i, _p, _p]),
    "ictc_species_linear": (_i, [_p, _i64, _i64, _i, _p, _i, _p, _p, _i, _p, _i64, _p]),
    "ictc_species_outer_workspace_bytes": (_i64, [_i64, _i, _i, _i]),
    "ictc_species_outer": (_i, [_p, _i64, _p, _i64, _i64, _i, _i, _p, _p, _i, _p, _p, _i64, _p]),
    "ictc_gemm_tn": (_i, [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p]),
    "ictc_edge_unit": (_i, [_i, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p]),
    "ictc_gemm_tn_grouped": (_i, [_p, _i64, _i64, _i, _i64, _p, _i64, _i64, _i, _i64, _i64, _i, _i64, _i64, _p, _p,
                                  _i64, _p]),
    "ictc_edge_geometry_fwd": (_i, [_p, _p, _p, _p, _i64, _i64, ctypes.c_float, _p, _p, _p, _p]),
    "ictc_edge_geometry_bwd": (_i, [_p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p]),
    "ictc_edge_vector_bwd": (_i, [_p, _i64, _i64, _p, _p, _p, _p, _p, _p]),
    "ictc_shift_vectors": (_i, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _p]),
    "ictc_edge_harmonics_fwd": (_i, [_p, _p, _p, _p, _i64, _i64, ctypes.c_float, _i, _p, _p, _p, _p, _p]),
    "ictc_edge_harmonics_bwd": (_i, [_p, _p, _p, _p, _p, _p, _i64, _i, _p, _p]),
    "ictc_radial_mlp_fwd": (_i, [_p, _i64, _i, _i, ctypes.c_float, _i, _p, _p, _p, ctypes.c_float, _p, _p]),
    "ictc_radial_mlp_tangent_fwd": (_i, [_p, _i64, _i, _i, ctypes.c_float, _i, _p, _p, _p, ctypes.c_float, _p, _p,
                                         _p]),
    "ictc_radial_mlp_bwd": (_i, [_p, _i64, _i, _i, ctypes.c_float, _i, _p, _p, _p, ctypes.c_float, _p, _p, _p, _p,
                                 _p, _p, _p, _p]),
    "ictc_radial_mlp_bwd2": (_i, [_p, _i64, _i, _i, ctypes.c_float, _i, _p, _p, _p, ctypes.c_float, _p, _p, _p, _p,
                                  _p, _p, _p, _p, _p, _p, _p, _p]),
    "ictc_sc_terms": (_i, [_i, _i, _i]),
    "ictc_sc_shape": (_i, [_i, _i, _i, _p, _p]),
    "ictc_sc_workspace_bytes": (_i64, [_i, _i, _i, _i, _i64, _i]),
    "ictc_sc_fwd": (_i, [_i, _i, _i, _i, _p, _p, _i, _p, _i64, _p, _p]),
    "ictc_sc_bwd_x": (_i, [_i, _i, _i, _i, _p, _p, _i, _p, _i64, _p, _p, _p]),
    "ictc_sc_bwd_w": (_i, [_i, _i, _i, _i, _p, _i, _i64, _p, _p, _p, _p, _p, _i64, _p]),
    "ictc_sc_jvp": (_i, [_i, _i, _i, _i, _p, _p, _i, _p, _i64, _p, _p, _p]),
    "ictc_sc_hvp": (_i, [_i, _i, _i, _i, _p, _p, _i, _p, _i64, _p, _p, _p, _p]),
    "ictc_sc_bwd_w_jvp": (_i, [_i, _i, _i, _i, _p, _i, _i64, _p, _p, _p, _p, _p, _p, _i64, _p]),
}


class NativeError(RuntimeError):
    """A C-ABI call returned a nonzero status."""


def library_path() -> str:
    return _LIB_PATH


def lib():
    """Load (once) and return the ctypes library; raises if it was not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.isfile(_LIB_PATH):
                    raise RuntimeError(
                        f"libictc_mi355x.so is not built ({_LIB_PATH}); run "
                        "`python ictc-o3-hp-k100_amd/csrc/build.py` (or __graft_entry__.build())")
                handle = ctypes.CDLL(_LIB_PATH)
                for name, (res, args) in _SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype, fn.argtypes = res, args
                _lib = handle
    return _lib


def exported_symbols():
    return tuple(_SIGNATURES)


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().ictc_last_error().decode(errors="replace")
        if rc in (-1, -2):
            raise ValueError(f"{name}: {msg}")
        raise NativeError(f"{name} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    if t.device.type != "cuda":
        raise ValueError("ICTC MI355X kernels require tensors on a ROCm (cuda) device")
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def tp_shape(li: int, le: int, lo: int):
    P, NO = _i(), _i()
    call("ictc_tp_shape", li, le, lo, ctypes.byref(P), ctypes.byref(NO))
    return P.value, NO.value
