"""gfh_gemv_w8_noalloc: the allocation-free form of the int8 decode GEMV,
called through the C ABI and checked against gfh_gemv_w8 (the same kernels,
so bit for bit) and against the oracle's dequantize + matmul (the GEMM bound),
on two calls in a row -- the second with a smaller input -- and with the
library's own call in between.  Sizes beyond its fixed scratch are rejected
before anything is launched."""
import numpy as np
import pytest

from _util import gemm_tol, to_dev, to_np

pytestmark = pytest.mark.gpu


def _case(dev, b, k, n, seed):
    from ghostflow_hip import synth
    from oracle import oracle as O
    x = synth.normal((b, k), seed=seed, tensor_id=0)
    w = synth.normal((k, n), 0.0, 0.02, seed=seed, tensor_id=1)
    q, s, z = O.quantize_per_channel(w, False)
    ref = O.matmul(x, O.dequantize(q, s, z))
    return [to_dev(a, dev) for a in (x, q, s, z)], ref, x, O.dequantize(q, s, z)


def _call(name, args, b, k, n, dev):
    import torch
    import ghostflow_hip
    L = ghostflow_hip.lib()
    x, q, s, z = args
    y = torch.full((b, n), float("nan"), device=dev)
    rc = getattr(L, name)(x.data_ptr(), q.data_ptr(), s.data_ptr(), z.data_ptr(), y.data_ptr(), b, k, n,
                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.gfh_last_error()
    torch.cuda.synchronize()
    return to_np(y)


@pytest.mark.parametrize("first,second", [((8, 4096, 14336), (3, 2048, 2560)), ((4, 11008, 4096), (1, 4096, 512))])
def test_noalloc_matches_gemv_w8_two_calls(torch_dev, first, second):
    """Two noalloc calls in a row (the second smaller, so it reads a scratch
    array that still holds the first call's partials), each bit-identical to
    gfh_gemv_w8 on the same inputs and within the GEMM bound of the oracle.
    Both shapes split K, so the partials and counters are in use."""
    for (b, k, n), seed in ((first, 1), (second, 2)):
        args, ref, x, dw = _case(torch_dev, b, k, n, seed)
        got = _call("gfh_gemv_w8_noalloc", args, b, k, n, torch_dev)
        lib_y = _call("gfh_gemv_w8", args, b, k, n, torch_dev)
        np.testing.assert_array_equal(got.view(np.uint32), lib_y.view(np.uint32))
        assert np.abs(got - ref).max() <= gemm_tol(k, x, dw)
        again = _call("gfh_gemv_w8_noalloc", args, b, k, n, torch_dev)
        np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))


def test_noalloc_batch_groups_and_unsplit(torch_dev):
    """b = 19 runs three batch groups that share the scratch in turn; a
    short K (one slice) uses no scratch at all."""
    for b, k, n in ((19, 3000, 1000), (2, 100, 4096)):
        args, ref, x, dw = _case(torch_dev, b, k, n, 5)
        got = _call("gfh_gemv_w8_noalloc", args, b, k, n, torch_dev)
        np.testing.assert_array_equal(got.view(np.uint32), _call("gfh_gemv_w8", args, b, k, n, torch_dev).view(np.uint32))
        assert np.abs(got - ref).max() <= gemm_tol(k, x, dw)


def test_noalloc_rejects_beyond_its_scratch(torch_dev):
    """b = 8, k = 4096, n = 70000 needs 4 slices x 8 rows x 70000 columns of
    partials (8.96 MB > 8 MiB): GFH_INVALID_SHAPE, y untouched."""
    import torch
    import ghostflow_hip
    L = ghostflow_hip.lib()
    b, k, n = 8, 4096, 70000
    x = torch.zeros((b, k), device=torch_dev)
    q = torch.zeros((k, n), dtype=torch.int8, device=torch_dev)
    s = torch.ones((k,), device=torch_dev)
    y = torch.full((b, n), 7.0, device=torch_dev)
    rc = L.gfh_gemv_w8_noalloc(x.data_ptr(), q.data_ptr(), s.data_ptr(), None, y.data_ptr(), b, k, n,
                               torch.cuda.current_stream().cuda_stream)
    assert rc == 1
    assert b"scratch" in L.gfh_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
