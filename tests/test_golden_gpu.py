"""GPU: the HIP path against the committed golden fixtures (the oracle's
outputs on seeded inputs).  Integer results (codes, scales, zero points,
int32 accumulators) must match bit for bit; fp32 results within the
north-star bounds."""
import os

import numpy as np
import pytest

from _util import gemm_tol, to_dev, to_np

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GEMM_SHAPES = [(1, 1, 1), (7, 5, 3), (33, 17, 29), (64, 64, 64), (128, 96, 200)]


def load(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def test_gemm_and_linear(torch_dev):
    gh, fx = _gh(), load("gemm")
    for m, k, n in GEMM_SHAPES:
        tag = f"{m}x{k}x{n}"
        a, b, c = fx[f"a_{tag}"], fx[f"b_{tag}"], fx[f"c_{tag}"]
        got = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
        assert np.abs(got - c).max() <= gemm_tol(k, a, b), tag
    x, w, b, y = fx["linear_x"], fx["linear_w"], fx["linear_b"], fx["linear_y"]
    got = to_np(gh.linear(to_dev(x, torch_dev), to_dev(w, torch_dev), to_dev(b, torch_dev)))
    assert np.abs(got - y).max() <= gemm_tol(64, x, w)


def test_quantization_bit_exact(torch_dev):
    gh, fx = _gh(), load("quant")
    names = sorted({k.rsplit("_", 1)[0] for k in fx.files if k.endswith("_kind")})
    assert names
    for nm in names:
        per_channel, sym = (bool(v) for v in fx[f"{nm}_kind"])
        x = to_dev(fx[f"{nm}_x"], torch_dev)
        if per_channel:
            q, s, z = gh.quantize_per_channel(x, symmetric=sym)
        else:
            q, s, z = gh.quantize_per_tensor(x, symmetric=sym)
        np.testing.assert_array_equal(to_np(q), fx[f"{nm}_q"], err_msg=nm)
        np.testing.assert_array_equal(to_np(s).view(np.uint32), fx[f"{nm}_s"].view(np.uint32), err_msg=nm)
        np.testing.assert_array_equal(to_np(z), fx[f"{nm}_z"], err_msg=nm)
        deq = to_np(gh.dequantize(q, s, z))
        np.testing.assert_array_equal(deq, fx[f"{nm}_deq"], err_msg=nm)


def test_qlinear_bit_exact(torch_dev):
    gh, fx = _gh(), load("qlinear")
    qw, sw, bias = (to_dev(fx[k], torch_dev) for k in ("qw", "sw", "bias"))
    for m in (1, 5):
        for row in (False, True):
            p = f"m{m}_row_" if row else f"m{m}_"
            qx, sx, zx = (to_dev(fx[p + k], torch_dev) for k in ("qx", "sx", "zx"))
            y, acc = gh.qlinear(qx, sx, zx, qw, sw, x_per_row=row, bias=None if row else bias,
                                want_acc=True)
            np.testing.assert_array_equal(to_np(acc), fx[p + "acc"])
            np.testing.assert_array_equal(to_np(y), fx[p + "y"])


def test_gemv(torch_dev):
    gh, fx = _gh(), load("gemv")
    x = to_dev(fx["x"], torch_dev)
    y = to_np(gh.gemv_f32(x, to_dev(fx["w"], torch_dev)))
    assert np.abs(y - fx["y"]).max() <= gemm_tol(64, fx["x"], fx["w"])
    for q, s, z, ref in (("qw", "s", "z", "y_w8"), ("qa", "sa", "za", "y_w8_asym")):
        got = to_np(gh.gemv_w8(x, to_dev(fx[q], torch_dev), to_dev(fx[s], torch_dev),
                               to_dev(fx[z], torch_dev)))
        assert np.abs(got - fx[ref]).max() <= gemm_tol(64, fx["x"], np.abs(fx["w"]).max() * 1.01)


def test_sdpa_and_softmax(torch_dev):
    gh, fx = _gh(), load("sdpa")
    for s in (8, 37):
        q, k, v = (to_dev(fx[f"s{s}_{t}"], torch_dev) for t in "qkv")
        o, w = gh.sdpa(q, k, v, want_weights=True)
        ref = fx[f"s{s}_out"]
        assert np.abs(to_np(o) - ref).max() <= 1e-4 * np.abs(ref).max()
        np.testing.assert_allclose(to_np(w), fx[f"s{s}_weights"], rtol=1e-4, atol=1e-7)
        oc = to_np(gh.sdpa(q, k, v, causal=True))
        ref = fx[f"s{s}_causal_out"]
        assert np.abs(oc - ref).max() <= 1e-4 * np.abs(ref).max()
    y = to_np(gh.softmax_lastdim(to_dev(fx["softmax_x"], torch_dev)))
    np.testing.assert_allclose(y, fx["softmax_y"], rtol=1e-4, atol=1e-12)
