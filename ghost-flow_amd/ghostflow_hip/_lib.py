"""ctypes declarations of the C ABI in include/ghostflow_hip.h and of the
Tensor-level API in include/ghostflow.h.

The shared library is built in-tree (ghost-flow_amd/Makefile) and loaded from
this directory.  There is no fallback: if the library is missing the import
of any compute entry point fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libghostflow_hip.so")

# Status codes (GhostFlowError, ghostflow-ffi/src/lib.rs:27-35).
SUCCESS = 0
INVALID_SHAPE = 1
INVALID_DATA = 2
NULL_POINTER = 3
ALLOCATION_FAILED = 4
COMPUTATION_FAILED = 5
UNKNOWN = 99
STATUS_NAMES = {
    SUCCESS: "Success",
    INVALID_SHAPE: "InvalidShape",
    INVALID_DATA: "InvalidData",
    NULL_POINTER: "NullPointer",
    ALLOCATION_FAILED: "AllocationFailed",
    COMPUTATION_FAILED: "ComputationFailed",
    UNKNOWN: "Unknown",
}

_p = C.c_void_p
_i = C.c_int
_i64 = C.c_int64
_f = C.c_float
_sz = C.c_size_t

# name -> (restype, argtypes); mirrors include/ghostflow_hip.h one to one.
SIGNATURES = {
    "gfh_init": (_i, []),
    "gfh_shutdown": (_i, []),
    "gfh_last_error": (C.c_char_p, []),
    "gfh_version": (C.c_char_p, []),
    "gfh_set_pointer_checks": (_i, [_i]),
    "gfh_sgemm": (_i, [_i, _i, _i64, _i64, _i64, _f, _p, _i64, _p, _i64, _f, _p, _i64, _p, _p]),
    "gfh_sgemm_strided_batched": (_i, [_i, _i, _i64, _i64, _i64, _f, _p, _i64, _i64, _i64, _p, _i64,
                                       _i64, _i64, _f, _p, _i64, _i64, _i64, _p, _p]),
    "gfh_matmul_backward_f32": (_i, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "gfh_quantize_i8_per_channel": (_i, [_p, _i64, _i64, _i, _p, _p, _p, _p]),
    "gfh_quantize_i8_per_tensor": (_i, [_p, _i64, _i, _p, _p, _p, _p, _sz, _p]),
    "gfh_quantize_i8_per_tensor_workspace_size": (_sz, [_i64]),
    "gfh_dequantize_i8": (_i, [_p, _i64, _i64, _p, _p, _i64, _p, _p]),
    "gfh_qweight_rowsum": (_i, [_p, _i64, _i64, _p, _p]),
    "gfh_qlinear_i8": (_i, [_p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "gfh_qlinear_dynamic_i8_workspace_size": (_sz, [_i64, _i64]),
    "gfh_qlinear_dynamic_i8": (_i, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _sz, _p]),
    "gfh_gemv_f32": (_i, [_p, _p, _p, _i64, _i64, _i64, _p]),
    "gfh_gemv_w8": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "gfh_gemv_w8_noalloc": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "gfh_softmax_lastdim_f32": (_i, [_p, _p, _i64, _i64, _p]),
    "gfh_flash_attention_workspace_size": (_sz, [_i64, _i64, _i64]),
    "gfh_flash_attention_f32": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _f, _p, _sz, _p]),
    "gfh_sdpa_f32": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f, _i, _p, _i64, _p]),
    "gfh_kv_attention_f32": (_i, [_p, _i64, _p, _p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f,
                                  _i, _p, _i64, _p]),
    "gfh_mha_workspace_size": (_sz, [_i64, _i64, _i64]),
    "gfh_mha_forward_with_cache_f32": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p,
                                            _i64, _i, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _sz, _p]),
    "gfh_silu_mul_f32": (_i, [_p, _p, _p, _i64, _p]),
    "gfh_state_dict_open": (_i, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "gfh_state_dict_close": (None, [_p]),
    "gfh_state_dict_count": (_i64, [_p]),
    "gfh_state_dict_entry": (_i, [_p, _i64, C.POINTER(C.c_char_p), C.POINTER(_i), C.POINTER(_i), C.POINTER(_i),
                                  C.POINTER(_i64), _i, C.POINTER(_i64)]),
    "gfh_state_dict_find": (_i64, [_p, C.c_char_p]),
    "gfh_state_dict_read_f32": (_i, [_p, _i64, _p, _p]),
    "gfh_state_dict_read_q8": (_i, [_p, _i64, _p, _p, _p, _p]),
    "gfh_state_dict_save": (_i, [C.c_char_p, _i, _p, _i64, _p]),
    "gfh_swiglu_f32_workspace_size": (_sz, [_i64, _i64]),
    "gfh_swiglu_f32": (_i, [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "gfh_swiglu_i8_workspace_size": (_sz, [_i64, _i64, _i64]),
    "gfh_swiglu_i8": (_i, [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                           _sz, _p]),
}

# The Tensor-level API of include/ghostflow.h (ghostflow-ffi/src/lib.rs).
_up = C.POINTER(C.c_size_t)
_tp = C.c_void_p
TENSOR_SIGNATURES = {
    "ghostflow_init": (_i, []),
    "ghostflow_version": (_p, []),
    "ghostflow_free_string": (None, [_p]),
    "ghostflow_tensor_create": (_i, [C.POINTER(C.c_float), _sz, _up, _sz, C.POINTER(_tp)]),
    "ghostflow_tensor_zeros": (_i, [_up, _sz, C.POINTER(_tp)]),
    "ghostflow_tensor_ones": (_i, [_up, _sz, C.POINTER(_tp)]),
    "ghostflow_tensor_free": (None, [_tp]),
    "ghostflow_tensor_shape": (_i, [_tp, _up, C.POINTER(C.c_size_t)]),
    "ghostflow_tensor_data": (_i, [_tp, C.POINTER(C.c_float), C.POINTER(C.c_size_t)]),
    "ghostflow_tensor_add": (_i, [_tp, _tp, C.POINTER(_tp)]),
    "ghostflow_tensor_mul": (_i, [_tp, _tp, C.POINTER(_tp)]),
    "ghostflow_tensor_matmul": (_i, [_tp, _tp, C.POINTER(_tp)]),
    "ghostflow_tensor_reshape": (_i, [_tp, _up, _sz, C.POINTER(_tp)]),
    "ghostflow_get_last_error": (C.c_char_p, []),
}

_lib = None


class TensorEntry(C.Structure):
    """gfh_tensor_entry (include/ghostflow_hip.h)."""
    _fields_ = [("name", C.c_char_p), ("kind", C.c_int), ("dtype", C.c_int), ("ndim", C.c_int),
                ("dims", C.POINTER(C.c_int64)), ("data", C.c_void_p), ("scales", C.c_void_p),
                ("zero_points", C.c_void_p), ("nscales", C.c_int64)]


def load():
    """Load libghostflow_hip.so and declare every exported signature."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(or make -C ghost-flow_amd) first")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in list(SIGNATURES.items()) + list(TENSOR_SIGNATURES.items()):
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib
