"""ctypes helpers for the Tensor-level C API (include/ghostflow.h)."""
import ctypes as C

import numpy as np

SUCCESS, INVALID_SHAPE, INVALID_DATA, NULL_POINTER, ALLOCATION_FAILED, COMPUTATION_FAILED = 0, 1, 2, 3, 4, 5


_L = None


def lib():
    global _L
    if _L is None:
        from ghostflow_hip import _lib as L
        _L = L.load()
    return _L


def dims(shape):
    arr = (C.c_size_t * max(len(shape), 1))(*shape)
    return arr, len(shape)


class T:
    """Owns one GhostFlowTensor handle."""

    def __init__(self, handle):
        self.h = handle

    def free(self):
        if self.h:
            lib().ghostflow_tensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:  # interpreter shutdown
            pass

    def shape(self):
        buf = (C.c_size_t * 32)()
        nd = C.c_size_t(99)
        assert lib().ghostflow_tensor_shape(self.h, buf, C.byref(nd)) == SUCCESS
        return tuple(buf[i] for i in range(nd.value))

    def numpy(self):
        shp = self.shape()
        n = int(np.prod(shp)) if shp else 1
        out = np.full(max(n, 1), np.nan, np.float32)
        ln = C.c_size_t(12345)
        rc = lib().ghostflow_tensor_data(self.h, out.ctypes.data_as(C.POINTER(C.c_float)), C.byref(ln))
        assert rc == SUCCESS, lib().ghostflow_get_last_error()
        assert ln.value == n
        return out[:n].reshape(shp)


def create(a):
    a = np.array(a, np.float32, order="C")  # keeps 0-d shapes (ascontiguousarray makes them 1-d)
    d, nd = dims(a.shape)
    h = C.c_void_p()
    flat = a.reshape(-1) if a.size else np.zeros(1, np.float32)
    rc = lib().ghostflow_tensor_create(flat.ctypes.data_as(C.POINTER(C.c_float)), a.size, d, nd, C.byref(h))
    assert rc == SUCCESS, lib().ghostflow_get_last_error()
    return T(h.value)


def call2(name, a, b):
    """(status, T or None) of ghostflow_tensor_<name>(a, b, &out)."""
    h = C.c_void_p()
    rc = getattr(lib(), "ghostflow_tensor_" + name)(a.h, b.h, C.byref(h))
    return rc, (T(h.value) if rc == SUCCESS else None)
