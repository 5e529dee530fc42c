"""CPU tests of the C ABI: the library loads, exports every symbol the header
declares, and rejects bad arguments on the host before touching a device."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ghostflow_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"GFH_API\s+[\w\s\*]+?\b(gfh_\w+)\s*\(", text)))


def _lib():
    from ghostflow_hip import _lib as L
    return L.load()


def test_header_declares_entry_points():
    names = _declared()
    for must in ("gfh_sgemm", "gfh_qlinear_i8", "gfh_gemv_f32", "gfh_gemv_w8", "gfh_sdpa_f32",
                 "gfh_quantize_i8_per_channel", "gfh_quantize_i8_per_tensor", "gfh_dequantize_i8",
                 "gfh_softmax_lastdim_f32", "gfh_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    from ghostflow_hip import _lib as L
    assert sorted(L.SIGNATURES) == _declared()


def test_version_and_last_error():
    lib = _lib()
    assert b"gfx950" in lib.gfh_version()
    assert lib.gfh_last_error() is not None


# Host-side validation: these fail before any device call, so they run on CPU.

def _fake(n=4096):
    """A host buffer address; never dereferenced because validation fails first."""
    buf = (C.c_char * n)()
    return C.cast(buf, C.c_void_p), buf


def test_sgemm_rejects_negative_dims():
    lib = _lib()
    rc = lib.gfh_sgemm(0, 0, -1, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4, None, None)
    assert rc == 1
    assert b"dims" in lib.gfh_last_error()


def test_sgemm_rejects_small_leading_dim():
    lib = _lib()
    rc = lib.gfh_sgemm(0, 0, 8, 8, 8, 1.0, None, 4, None, 8, 0.0, None, 8, None, None)
    assert rc == 1
    assert b"leading dimension" in lib.gfh_last_error()


def test_sgemm_null_operands():
    lib = _lib()
    rc = lib.gfh_sgemm(0, 0, 8, 8, 8, 1.0, None, 8, None, 8, 0.0, None, 8, None, None)
    assert rc == 3
    assert b"NULL" in lib.gfh_last_error()


def test_sgemm_empty_is_noop():
    lib = _lib()
    assert lib.gfh_sgemm(0, 0, 0, 8, 8, 1.0, None, 8, None, 8, 0.0, None, 8, None, None) == 0


def test_sgemm_rejects_host_memory():
    lib = _lib()
    p, keep = _fake(8 * 8 * 4)
    rc = lib.gfh_sgemm(0, 0, 8, 8, 8, 1.0, p, 8, p, 8, 0.0, p, 8, None, None)
    assert rc in (2, 5)  # not device memory (InvalidData) / no device (ComputationFailed)


def test_qlinear_k_bound_and_outputs():
    lib = _lib()
    assert lib.gfh_qlinear_i8(None, None, None, 0, None, None, None, None, None, None, 4, 4, 70000, None) == 1
    assert lib.gfh_qlinear_i8(None, None, None, 0, None, None, None, None, None, None, 4, 4, 64, None) == 3


def test_qlinear_dynamic_rules():
    """gfh_qlinear_dynamic_i8 validates on the host before any device work:
    the exact-int32 K bound, the required y / w_rowsum, element counts
    whose byte sizes would overflow, and the workspace size query."""
    lib = _lib()
    f = lib.gfh_qlinear_dynamic_i8
    assert f(None, None, None, None, None, None, 4, 4, 70000, None, 0, None) == 1   # K beyond 65793
    assert f(None, None, None, None, None, None, 4, 4, 64, None, 0, None) == 3      # y, w_rowsum NULL
    y = C.c_void_p(16)
    assert f(None, None, None, y, None, y, 2**31 - 1, 2**31 - 1, 64, None, 0, None) == 1  # m*n bytes overflow
    assert f(None, None, None, y, None, y, 0, 16, 64, None, 0, None) == 0             # empty: no work
    assert lib.gfh_qlinear_dynamic_i8_workspace_size(0, 64) == 0
    assert lib.gfh_qlinear_dynamic_i8_workspace_size(4, 4096) >= 4 * 4096


def test_gemv_batch_limit():
    lib = _lib()
    assert lib.gfh_gemv_f32(None, None, None, 65, 16, 16, None) == 1
    assert lib.gfh_gemv_w8(None, None, None, None, None, 65, 16, 16, None) == 1
    # k * n elements whose byte size would overflow
    big = 2**31 - 1
    assert lib.gfh_gemv_f32(None, None, None, 1, big, big, None) == 1
    assert lib.gfh_gemv_w8(None, None, None, None, None, 1, big, big, None) == 1


def test_flash_attention_shape_rules():
    """FlashAttention::forward's host checks: block sizes must be positive
    (the reference's step_by(0) panics), at most 8192 key blocks; the
    workspace size is batch * seq_len_q * seq_len_k floats."""
    lib = _lib()
    args = (None, None, None, None, 1, 4, 4, 8)
    assert lib.gfh_flash_attention_f32(*args, 0, 64, 0, 1.0, None, 0, None) == 1
    assert b"block sizes" in lib.gfh_last_error()
    assert lib.gfh_flash_attention_f32(*args, 64, -1, 0, 1.0, None, 0, None) == 1
    assert lib.gfh_flash_attention_f32(None, None, None, None, 1, 4, 8193, 8, 64, 1, 0, 1.0, None, 0, None) == 1
    assert b"key blocks" in lib.gfh_last_error()
    assert lib.gfh_flash_attention_f32(*args, 64, 64, 0, 1.0, None, 0, None) == 3  # NULL q
    assert lib.gfh_flash_attention_workspace_size(3, 5, 7) == 3 * 5 * 7 * 4
    assert lib.gfh_flash_attention_workspace_size(3, 5, 0) == 0


def test_sdpa_shape_rules():
    lib = _lib()
    # head_dim must be a multiple of 4 in [4,128]
    assert lib.gfh_sdpa_f32(None, None, None, None, None, 1, 1, 8, 8, 130, 1.0, 0, None, 0, None) == 1
    assert lib.gfh_sdpa_f32(None, None, None, None, None, 1, 1, 8, 8, 6, 1.0, 0, None, 0, None) == 1
    # causal needs sq == skv
    assert lib.gfh_sdpa_f32(None, None, None, None, None, 1, 1, 8, 9, 16, 1.0, 1, None, 0, None) == 1
    assert b"gfh_flash_attention_f32" in lib.gfh_last_error()  # the documented route for top-left causal
    # missing tensors
    assert lib.gfh_sdpa_f32(None, None, None, None, None, 1, 1, 8, 8, 16, 1.0, 1, None, 0, None) == 3


def test_dequantize_scale_count():
    lib = _lib()
    assert lib.gfh_dequantize_i8(None, 4, 4, None, None, 3, None, None) == 1


def test_python_wrapper_shape_mismatch():
    torch = pytest.importorskip("torch")
    import ghostflow_hip as gh
    from ghostflow_hip.ops import GhostFlowError
    a = torch.zeros(2, 3)
    with pytest.raises(GhostFlowError):
        gh.matmul(a, torch.zeros(4, 2))


def test_kv_attention_rejects_bad_shapes():
    lib = _lib()
    p, _keep = _fake()
    # head_dim not a multiple of 4
    assert lib.gfh_kv_attention_f32(p, 12, p, p, 8, 12, p, 12, None, 1, 2, 1, 8, 6, 1.0, 0, None, 0, None) == 1
    assert b"head_dim" in lib.gfh_last_error()
    # kv_len beyond the cache capacity
    assert lib.gfh_kv_attention_f32(p, 16, p, p, 8, 16, p, 16, None, 1, 2, 1, 9, 8, 1.0, 0, None, 0, None) == 1
    assert b"capacity" in lib.gfh_last_error()
    # leading dimension below h * d
    assert lib.gfh_kv_attention_f32(p, 8, p, p, 8, 16, p, 16, None, 1, 2, 1, 8, 8, 1.0, 0, None, 0, None) == 1
    assert b"ldq" in lib.gfh_last_error()
    # causal with more queries than keys
    assert lib.gfh_kv_attention_f32(p, 16, p, p, 8, 16, p, 16, None, 1, 2, 4, 3, 8, 1.0, 1, None, 0, None) == 1
    assert b"causal" in lib.gfh_last_error()
    # a key leading dimension whose extent over kv_len rows would overflow
    big = 2**62
    assert lib.gfh_kv_attention_f32(p, 16, p, p, 8, big, p, 16, None, 1, 2, 1, 8, 8, 1.0, 0, None, 0, None) == 1
    assert b"overflows" in lib.gfh_last_error()
    # a mask whose byte size would overflow
    assert lib.gfh_kv_attention_f32(p, 16, p, p, 8, 16, p, 16, None, 1, 2, 1, 8, 8, 1.0, 0, p, big, None) == 1
    assert b"mask_numel" in lib.gfh_last_error()
    assert lib.gfh_sdpa_f32(p, p, p, p, None, 1, 1, 8, 8, 16, 1.0, 0, p, big, None) == 1
    assert b"mask_numel" in lib.gfh_last_error()
    w = [p] * 8  # wq, bq, wk, bk, wv, bv, wo, bo
    assert lib.gfh_mha_forward_with_cache_f32(p, p, p, *w, p, p, 16, 0, p, big, 0, p, None, 1, 1, 1, 16, 2,
                                              None, 0, None) == 1
    assert b"mask_numel" in lib.gfh_last_error()


def test_swiglu_rejects_bad_shapes():
    lib = _lib()
    p, _keep = _fake()
    assert lib.gfh_silu_mul_f32(p, p, p, -1, None) == 1
    assert lib.gfh_silu_mul_f32(None, None, None, 0, None) == 0  # empty is a no-op
    assert lib.gfh_swiglu_f32(p, -1, 16, 16, p, None, p, None, p, None, p, None, None, 0, None) == 1
    assert b"out of range" in lib.gfh_last_error()
    assert lib.gfh_swiglu_f32(None, 0, 16, 16, None, None, None, None, None, None, None, None, None, 0,
                              None) == 0
    # int8 rows must be whole 16-byte groups
    args = [p] * 12
    assert lib.gfh_swiglu_i8(p, 2, 24, 32, *args, p, None, None, 0, None) == 1
    assert b"multiples of 16" in lib.gfh_last_error()
    assert lib.gfh_swiglu_i8(p, 2, 16, 70000 * 16, *args, p, None, None, 0, None) == 1
    assert b"exact-int32" in lib.gfh_last_error()
    # host memory is not device memory
    assert lib.gfh_swiglu_i8(p, 2, 16, 32, *args, p, None, None, 0, None) != 0


def test_swiglu_workspace_sizes():
    lib = _lib()
    assert lib.gfh_swiglu_f32_workspace_size(4, 100) >= 2 * 4 * 100 * 4
    # fused gate/up (hidden % 64 == 0): x codes, h, h codes
    assert lib.gfh_swiglu_i8_workspace_size(4, 64, 96) >= 4 * 64 + 4 * 96 * 4 + 4 * 96
    # unfused (hidden = 80): gate and up in fp32 as well
    assert lib.gfh_swiglu_i8_workspace_size(70, 80, 96) >= 70 * 80 + 2 * 70 * 96 * 4 + 70 * 96
    # shapes the entry points reject as out of range size to 0
    assert lib.gfh_swiglu_i8_workspace_size(-1, -1, -1) == 0
    assert lib.gfh_swiglu_f32_workspace_size(2**40, 2**40) == 0
    assert lib.gfh_swiglu_i8_workspace_size(2**31 - 1, 2**31 - 1, 16) == 0
    assert lib.gfh_quantize_i8_per_tensor_workspace_size(2**41) == 0
    assert lib.gfh_flash_attention_workspace_size(2**33, 1, 1) == 0


def test_matmul_backward_rejects_bad_dims():
    lib = _lib()
    assert lib.gfh_matmul_backward_f32(None, None, None, -1, 2, 2, None, None, None) == 1
    assert b"matmul_backward" in lib.gfh_last_error()
    # nothing requested: no work, no pointer needed
    assert lib.gfh_matmul_backward_f32(None, None, None, 2, 2, 2, None, None, None) == 0
