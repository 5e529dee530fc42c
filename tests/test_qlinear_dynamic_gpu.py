"""gfh_qlinear_dynamic_i8: the INT8 linear on fp32 activations, x quantized
per tensor (asymmetric, DynamicQuantization::quantize_activation,
ghostflow-nn/src/quantization.rs:280-287) and multiplied with per-channel
weight codes.  Bar: bit-exact against the oracle's quantize_per_tensor +
qlinear_i8 (the a22 spec's epilogue), and against the library's own
quantize_per_tensor + qlinear.  m <= 4 runs as one launch (the INT8 kernel
quantizes x itself, including a K split over workgroups); larger m,
misaligned x and k % 16 != 0 take the two-launch form."""
import numpy as np
import pytest

from _util import to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _O():
    from oracle import oracle
    return oracle


CASES = [
    # (m, n, k, bias)
    (1, 11008, 4096, True),   # the decode shape, one launch
    (2, 300, 64, False),
    (3, 1040, 208, True),
    (4, 4096, 11008, True),   # K split over two workgroups per column block
    (1, 512, 65536, False),   # the largest K of the exact-int32 bound, 16 K-slices
    (4, 1000, 4096, True),
    (5, 2048, 4096, True),    # two launches from here on
    (64, 1000, 256, False),
    (300, 512, 1024, True),
    (3, 700, 200, True),      # k % 16 != 0: two launches
]


@pytest.mark.parametrize("m,n,k,bias", CASES)
def test_matches_quantize_then_qlinear(torch_dev, m, n, k, bias):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(m * 7 + n + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    x[0, 0] = 3.75  # a known max, so that the scale and zero point are exercised away from symmetry
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    b = rng.uniform(-0.01, 0.01, n).astype(np.float32) if bias else None
    qw, sw, _ = O.quantize_per_channel(w, True)
    dqw, dsw = to_dev(qw, torch_dev), to_dev(sw, torch_dev)
    rs = gh.qweight_rowsum(dqw)
    db = to_dev(b, torch_dev) if bias else None
    got = to_np(gh.qlinear_dynamic(to_dev(x, torch_dev), dqw, dsw, rs, bias=db))
    qx, sx, zx = O.quantize_per_tensor(x, False)
    ref, _ = O.qlinear_i8(qx, sx, zx, False, qw, sw, b, want_acc=False)
    np.testing.assert_array_equal(got, ref)
    qxd, sxd, zxd = gh.quantize_per_tensor(to_dev(x, torch_dev), symmetric=False)
    two, _ = gh.qlinear(qxd, sxd, zxd, dqw, dsw, w_rowsum=rs, bias=db)
    np.testing.assert_array_equal(got, to_np(two))


def test_misaligned_x_and_caller_workspace(torch_dev):
    """x 4 bytes past a 16-byte boundary at m = 2 (the two-launch form), with
    a caller workspace of exactly gfh_qlinear_dynamic_i8_workspace_size
    bytes; and the aligned call, which needs none."""
    import torch
    gh, O = _gh(), _O()
    m, n, k = 2, 1024, 4096
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qw, sw, _ = O.quantize_per_channel(rng.normal(0, 0.02, (n, k)).astype(np.float32), True)
    dqw, dsw = to_dev(qw, torch_dev), to_dev(sw, torch_dev)
    rs = gh.qweight_rowsum(dqw)
    buf = torch.zeros(m * k + 4, dtype=torch.float32, device=torch_dev)
    buf[1:1 + m * k] = to_dev(x.reshape(-1), torch_dev)
    xv = buf[1:1 + m * k].view(m, k)
    assert xv.data_ptr() % 16 == 4
    nbytes = int(gh._lib.load().gfh_qlinear_dynamic_i8_workspace_size(m, k))
    ws = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=torch_dev)
    got = to_np(gh.qlinear_dynamic(xv, dqw, dsw, rs, workspace=ws))
    qx, sx, zx = O.quantize_per_tensor(x, False)
    ref, _ = O.qlinear_i8(qx, sx, zx, False, qw, sw, None, want_acc=False)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(to_np(gh.qlinear_dynamic(to_dev(x, torch_dev), dqw, dsw, rs)), ref)


def test_nan_and_inf_activations(torch_dev):
    """Non-finite activations at m = 1: the min / max fold ignores NaN (as
    f32::min / max), an inf makes the scale inf and every code follows the
    reference's saturating casts -- the same codes as the quantize pass."""
    gh, O = _gh(), _O()
    m, n, k = 1, 512, 1024
    rng = np.random.default_rng(9)
    qw, sw, _ = O.quantize_per_channel(rng.normal(0, 0.02, (n, k)).astype(np.float32), True)
    dqw, dsw = to_dev(qw, torch_dev), to_dev(sw, torch_dev)
    rs = gh.qweight_rowsum(dqw)
    for special in (np.nan, np.inf):
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        x[0, 17] = special
        got = to_np(gh.qlinear_dynamic(to_dev(x, torch_dev), dqw, dsw, rs))
        qx, sx, zx = O.quantize_per_tensor(x, False)
        ref, _ = O.qlinear_i8(qx, sx, zx, False, qw, sw, None, want_acc=False)
        np.testing.assert_array_equal(got, ref)
