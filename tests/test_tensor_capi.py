"""CPU tests of the Tensor-level C API (include/ghostflow.h): every declared
entry point is exported, and the argument checks of ghostflow-ffi/src/lib.rs
(NullPointer, InvalidShape before any device work) hold without a GPU."""
import ctypes as C
import os
import re

from _capi import INVALID_SHAPE, NULL_POINTER, dims, lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ghostflow.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"GHOSTFLOW_API\s+[\w\s\*]+?\b(ghostflow_\w+)\s*\(", text)))


def test_header_declares_the_reference_entry_points():
    # ghostflow-ffi/src/lib.rs:60-337
    want = ["ghostflow_init", "ghostflow_version", "ghostflow_free_string", "ghostflow_tensor_create",
            "ghostflow_tensor_zeros", "ghostflow_tensor_ones", "ghostflow_tensor_free", "ghostflow_tensor_shape",
            "ghostflow_tensor_data", "ghostflow_tensor_add", "ghostflow_tensor_mul", "ghostflow_tensor_matmul",
            "ghostflow_tensor_reshape", "ghostflow_get_last_error"]
    assert _declared() == sorted(want)


def test_library_exports_and_signatures_cover_header():
    from ghostflow_hip import _lib as L
    L_ = lib()
    assert all(hasattr(L_, n) for n in _declared())
    assert sorted(L.TENSOR_SIGNATURES) == _declared()


def test_error_codes_match_reference():
    text = open(HEADER).read()
    for name, code in (("Success", 0), ("InvalidShape", 1), ("InvalidData", 2), ("NullPointer", 3),
                       ("AllocationFailed", 4), ("ComputationFailed", 5), ("Unknown", 99)):
        assert re.search(rf"\b{name}\s*=\s*{code}\b", text)


def test_version_string_round_trip():
    L_ = lib()
    p = L_.ghostflow_version()
    assert b"gfx950" in C.cast(p, C.c_char_p).value
    L_.ghostflow_free_string(p)


def test_null_arguments():
    L_ = lib()
    h = C.c_void_p()
    d, nd = dims((2, 2))
    data = (C.c_float * 4)()
    assert L_.ghostflow_tensor_create(None, 4, d, nd, C.byref(h)) == NULL_POINTER
    assert L_.ghostflow_tensor_create(data, 4, None, nd, C.byref(h)) == NULL_POINTER
    assert L_.ghostflow_tensor_create(data, 4, d, nd, None) == NULL_POINTER
    assert L_.ghostflow_tensor_zeros(None, 1, C.byref(h)) == NULL_POINTER
    assert L_.ghostflow_tensor_ones(d, nd, None) == NULL_POINTER
    n = C.c_size_t()
    assert L_.ghostflow_tensor_shape(None, (C.c_size_t * 4)(), C.byref(n)) == NULL_POINTER
    assert L_.ghostflow_tensor_data(None, data, C.byref(n)) == NULL_POINTER
    for op in ("add", "mul", "matmul"):
        assert getattr(L_, "ghostflow_tensor_" + op)(None, None, C.byref(h)) == NULL_POINTER
    assert L_.ghostflow_tensor_reshape(None, d, nd, C.byref(h)) == NULL_POINTER
    assert b"null" in L_.ghostflow_get_last_error()
    L_.ghostflow_tensor_free(None)  # a no-op, as Box::from_raw is skipped for null (lib.rs:166-171)


def test_create_length_must_match_shape():
    """Tensor::from_slice rejects data_len != numel (tensor.rs:38-46)."""
    L_ = lib()
    h = C.c_void_p()
    d, nd = dims((2, 3))
    data = (C.c_float * 8)()
    assert L_.ghostflow_tensor_create(data, 5, d, nd, C.byref(h)) == INVALID_SHAPE
    assert b"length" in L_.ghostflow_get_last_error()
    assert h.value is None
    d0, nd0 = dims(())  # a scalar: one element
    assert L_.ghostflow_tensor_create(data, 2, d0, nd0, C.byref(h)) == INVALID_SHAPE
