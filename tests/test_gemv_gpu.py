"""Decode GEMV (fp32 and int8 weights) on the GPU against the oracle
(Tensor::matmul at M = B; int8 = dequantize_int8 then matmul).  Bar: the
north-star GEMM bound max|err| <= 1e-4 * sqrt(K) * max|x| * max|w|;
bit-exact on integer-valued inputs."""
import numpy as np
import pytest

from _util import gemm_tol, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _O():
    from oracle import oracle
    return oracle


@pytest.mark.parametrize("b,k,n", [(1, 1, 1), (3, 64, 80), (1, 300, 999), (8, 1024, 1024), (5, 77, 1030),
                                   (13, 256, 512), (64, 128, 260), (8, 3000, 12300), (6, 4096, 16384),
                                   (1, 2500, 12800), (2, 4096, 13000), (4, 1000, 16000), (3, 2000, 25600),
                                   (9, 4096, 14336)])
def test_gemv_f32_integer_exact(torch_dev, b, k, n):
    """Integer data (exact in any order).  From (8, 3000, 12300) on, wide
    N: 192-256 strips in one slice (4096 rows of x in LDS for 8-row groups),
    2-4 slices with ragged K and a ragged last strip, and a second batch
    group of 1 row at b = 9."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(b * 7 + k + n)
    x = rng.integers(-8, 9, size=(b, k)).astype(np.float32)
    w = rng.integers(-8, 9, size=(k, n)).astype(np.float32)
    got = to_np(gh.gemv_f32(to_dev(x, torch_dev), to_dev(w, torch_dev)))
    np.testing.assert_array_equal(got, O.matmul(x, w))


@pytest.mark.parametrize("b,k,n", [(1, 256, 4096), (4, 4096, 14336), (8, 1000, 2048), (3, 2048, 13000)])
def test_gemv_f32_misaligned_x(torch_dev, b, k, n):
    """x 4 bytes past a 16-byte boundary (a view at element offset 1 of a
    larger buffer): the activations cannot be loaded 16 bytes at a time, so
    the kernel stages them for the whole slice instead of streaming them
    with the weights.  Integer data, exact; the aligned call agrees."""
    import torch
    gh, O = _gh(), _O()
    rng = np.random.default_rng(b * 31 + k + n)
    x = rng.integers(-8, 9, size=(b, k)).astype(np.float32)
    w = rng.integers(-8, 9, size=(k, n)).astype(np.float32)
    buf = torch.zeros(b * k + 4, dtype=torch.float32, device=torch_dev)
    buf[1:1 + b * k] = to_dev(x.reshape(-1), torch_dev)
    xv = buf[1:1 + b * k].view(b, k)
    assert xv.data_ptr() % 16 == 4
    dw = to_dev(w, torch_dev)
    got = to_np(gh.gemv_f32(xv, dw))
    np.testing.assert_array_equal(got, O.matmul(x, w))
    np.testing.assert_array_equal(got, to_np(gh.gemv_f32(to_dev(x, torch_dev), dw)))


def test_mv_reference_known_answer(torch_dev):
    """Tensor::mv [[1,2],[3,4]] . [1,2] = [5, 11] (matmul.rs:363-371), as
    x [1,2] . W^T with W^T = [[1,3],[2,4]]."""
    gh = _gh()
    x = np.array([[1, 2]], np.float32)
    wt = np.array([[1, 3], [2, 4]], np.float32)
    assert to_np(gh.gemv_f32(to_dev(x, torch_dev), to_dev(wt, torch_dev))).tolist() == [[5.0, 11.0]]


@pytest.mark.parametrize("b", [1, 4, 8])
def test_config4_fp32(torch_dev, b):
    """Config 4: W [4096,14336] ~ N(0,0.02), x [B,4096] ~ N(0,1)."""
    gh, O = _gh(), _O()
    k, n = 4096, 14336
    w = gh.normal((k, n), 0.0, 0.02, seed=0, tensor_id=1)
    x = gh.normal((b, k), seed=0, tensor_id=0)
    got = to_np(gh.gemv_f32(to_dev(x, torch_dev), to_dev(w, torch_dev)))
    ref = O.matmul(x, w)
    assert np.abs(got - ref).max() <= gemm_tol(k, x, w)


@pytest.mark.parametrize("b", [1, 4, 8])
@pytest.mark.parametrize("symmetric", [True, False])
def test_config4_int8(torch_dev, b, symmetric):
    """Config 4 int8: W [4096,14336] quantized per channel over dim 0 (one
    scale per k row); y vs dequantize(W) then matmul (the reference's path)."""
    gh, O = _gh(), _O()
    k, n = 4096, 14336
    w = gh.normal((k, n), 0.0, 0.02, seed=0, tensor_id=1)
    x = gh.normal((b, k), seed=0, tensor_id=0)
    q, s, z = gh.quantize_per_channel(to_dev(w, torch_dev), symmetric)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), q, s, z))
    rq, rs, rz = O.quantize_per_channel(w, symmetric)
    np.testing.assert_array_equal(to_np(q), rq)
    dw = O.dequantize(rq, rs, rz)
    ref = O.matmul(x, dw)
    assert np.abs(got - ref).max() <= gemm_tol(k, x, dw)


@pytest.mark.parametrize("b,k,n", [(2, 64, 80), (7, 333, 1001), (9, 1024, 2048)])
def test_gemv_w8_integer_exact(torch_dev, b, k, n):
    """Scales that are powers of two and small integer x: every product and
    partial sum is exact, so the result must match bit for bit."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(k + n)
    q = rng.integers(-128, 128, size=(k, n)).astype(np.int8)
    s = (2.0 ** rng.integers(-3, 2, size=k)).astype(np.float32)
    z = rng.integers(-5, 6, size=k).astype(np.int8)
    x = rng.integers(-4, 5, size=(b, k)).astype(np.float32)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(q, torch_dev), to_dev(s, torch_dev), to_dev(z, torch_dev)))
    ref = O.matmul(x, O.dequantize(q, s, z))
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("b,k,n", [(2, 1677, 33024), (3, 4136, 10000)])
def test_gemv_w8_refill_ring_integer_exact(torch_dev, b, k, n):
    """Shapes whose waves stream more weight blocks than they hold in
    registers.  [1677, 33024]: 129 strips x 2 slices, 4 waves per workgroup;
    the 1024-row slice gives 8 blocks per wave (one refill pass of the
    4-buffer ring), the 653-row slice 6, 6, 6 and 3 (refills that re-read
    the last block, and a wave with fewer blocks than buffers).  [4136,
    10000]: N % 16 != 0, so the byte-checked loads and their 2-buffer ring,
    8 blocks per wave."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(k * 3 + n)
    q = rng.integers(-128, 128, size=(k, n)).astype(np.int8)
    s = (2.0 ** rng.integers(-3, 2, size=k)).astype(np.float32)
    z = rng.integers(-5, 6, size=k).astype(np.int8)
    x = rng.integers(-4, 5, size=(b, k)).astype(np.float32)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(q, torch_dev), to_dev(s, torch_dev), to_dev(z, torch_dev)))
    ref = O.matmul(x, O.dequantize(q, s, z))
    np.testing.assert_array_equal(got, ref)


def test_gemv_w8_without_zero_points(torch_dev):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(1)
    q = rng.integers(-128, 128, size=(200, 300)).astype(np.int8)
    s = (2.0 ** rng.integers(-3, 2, size=200)).astype(np.float32)
    x = rng.integers(-4, 5, size=(3, 200)).astype(np.float32)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(q, torch_dev), to_dev(s, torch_dev)))
    np.testing.assert_array_equal(got, O.matmul(x, O.dequantize(q, s, np.zeros(200, np.int8))))


def test_split_k_counters_reset_across_calls_and_streams(torch_dev):
    """K is split over workgroups for the int8 GEMV; the last workgroup of
    each strip sums the slices and returns its arrival counter to zero.
    Repeated calls on the default stream and on a second stream must give
    identical (deterministic) results."""
    import torch
    gh = _gh()
    b, k, n = 3, 4096, 2048 + 96
    x = gh.normal((b, k), seed=12, tensor_id=0)
    w = gh.normal((k, n), 0.0, 0.02, seed=12, tensor_id=1)
    O = _O()
    qw, s, z = O.quantize_per_channel(w, False)
    dx, dq, ds, dz = (to_dev(a, torch_dev) for a in (x, qw, s, z))
    first = to_np(gh.gemv_w8(dx, dq, ds, dz))
    ref = O.matmul(x, O.dequantize(qw, s, z))
    assert np.abs(first - ref).max() <= gemm_tol(k, x, np.abs(w).max() * 1.01)
    for _ in range(3):
        np.testing.assert_array_equal(to_np(gh.gemv_w8(dx, dq, ds, dz)), first)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for _ in range(3):
            y2 = gh.gemv_w8(dx, dq, ds, dz)
    side.synchronize()
    np.testing.assert_array_equal(to_np(y2), first)


@pytest.mark.parametrize("b", [1, 4, 8])
def test_gemv_w8_activation_precision(torch_dev, b):
    """x * s is carried in full: its three f16 pieces hold 33 bits, more
    than the 24 of the fp32 product.  With exactly one non-zero weight per
    column, y[b, n] = x s (q - zp) has no sum over k, so the result carries
    only the rounding of x * s and of adding the three pieces' products:
    within 3 * 2^-24 relative of the exact value (two f16 pieces, 22 bits,
    are off by up to 2^-22 relative and fail this).  b = 8 takes the two-
    operand form, b <= 4 the one-operand form."""
    gh = _gh()
    rng = np.random.default_rng(40 + b)
    k, n = 1024, 512
    x = (rng.uniform(1.0, 2.0, size=(b, k)) * rng.choice([-1.0, 1.0], size=(b, k))).astype(np.float32)
    s = rng.uniform(0.5, 2.0, size=k).astype(np.float32)
    q = np.zeros((k, n), np.int8)
    rows = rng.integers(0, k, size=n)
    q[rows, np.arange(n)] = (rng.integers(1, 128, size=n) * rng.choice([-1, 1], size=n)).astype(np.int8)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(q, torch_dev), to_dev(s, torch_dev))).astype(np.float64)
    exact = x.astype(np.float64)[:, rows] * s.astype(np.float64)[rows] * q[rows, np.arange(n)].astype(np.float64)
    rel = np.abs(got - exact) / np.abs(exact)
    assert rel.max() <= 3.01 * 2.0 ** -24, rel.max()


def test_gemv_w8_wide_dynamic_range(torch_dev):
    """One K-slice whose |x s| spans more than 2^30 (log-uniform magnitudes
    from 2^-16 to 2^15, random signs): the f16 pieces of x s lose relative
    precision only far below the slice maximum, so the result must stay
    within the GEMM bound of the reference's dequantize + matmul."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(21)
    b, k, n = 3, 1024, 768
    _wide_range_case(gh, O, torch_dev, rng, b, k, n)
    _wide_range_case(gh, O, torch_dev, rng, b, k, 8192)


def _wide_range_case(gh, O, torch_dev, rng, b, k, n):
    mag = 2.0 ** rng.uniform(-16, 15, size=(b, k))
    x = (mag * rng.choice([-1.0, 1.0], size=(b, k))).astype(np.float32)
    x[0, 5], x[1, 7] = np.float32(2.0 ** 15), np.float32(2.0 ** -16)
    q = rng.integers(-128, 128, size=(k, n)).astype(np.int8)
    s = rng.uniform(0.5, 2.0, size=k).astype(np.float32)
    z = rng.integers(-5, 6, size=k).astype(np.int8)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(q, torch_dev), to_dev(s, torch_dev), to_dev(z, torch_dev)))
    dw = O.dequantize(q, s, z)
    ref = O.matmul(x, dw)
    assert np.abs(got - ref).max() <= gemm_tol(k, x, dw)


def test_gemv_w8_non_finite_activations(torch_dev):
    """An inf or NaN activation gives the reference's inf / NaN in its own
    batch row (x * dequantize(W): +-inf where the weight is non-zero, NaN
    where it is zero) and leaves the other batch rows of the same strip
    untouched -- the prescale of the slice ignores non-finite values."""
    gh, O = _gh(), _O()
    for n in (320, 8192):
        _non_finite_case(gh, O, torch_dev, np.random.default_rng(22), 4, 512, n)


def _non_finite_case(gh, O, torch_dev, rng, b, k, n):
    x = rng.standard_normal((b, k)).astype(np.float32)
    x[0, 10] = np.inf
    x[1, 20] = -np.inf
    x[2, 30] = np.nan
    q = rng.integers(-128, 128, size=(k, n)).astype(np.int8)
    q[10, :5] = 0  # zero weights under the inf: inf * 0 = NaN in the reference
    s = (2.0 ** rng.integers(-3, 2, size=k)).astype(np.float32)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(q, torch_dev), to_dev(s, torch_dev)))
    dw = O.dequantize(q, s, np.zeros(k, np.int8))
    ref = O.matmul(x, dw)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(np.isinf(got), np.isinf(ref))
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])
    assert np.abs(got[fin] - ref[fin]).max() <= gemm_tol(k, x[3], dw)
    assert np.isfinite(ref[3]).all()


@pytest.mark.parametrize("b,k,n", [(1, 4096, 8192), (3, 4100, 8208), (8, 5000, 14336), (13, 300, 10000),
                                   (2, 64, 32768), (5, 1, 9008), (4, 2000, 16400)])
def test_gemv_w8_wide_integer_exact(torch_dev, b, k, n):
    """Wide W (N >= 8192): ragged last strips (8208, 9008, 10000, 16400),
    K = 5000 in slices of unequal length, K = 1 and 64 (one short slice),
    batch groups of 8 (13).  Power-of-two scales and small integers: exact,
    so bit for bit against the oracle's dequantize + matmul."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(k * 5 + n + b)
    q = rng.integers(-128, 128, size=(k, n)).astype(np.int8)
    s = (2.0 ** rng.integers(-3, 2, size=k)).astype(np.float32)
    z = rng.integers(-5, 6, size=k).astype(np.int8)
    x = rng.integers(-4, 5, size=(b, k)).astype(np.float32)
    got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(q, torch_dev), to_dev(s, torch_dev), to_dev(z, torch_dev)))
    np.testing.assert_array_equal(got, O.matmul(x, O.dequantize(q, s, z)))
