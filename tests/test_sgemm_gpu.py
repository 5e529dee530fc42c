"""fp32 GEMM / Linear on the GPU against the oracle (matmul_blocked,
Linear::forward, batched_matmul restated from the reference).

Bars: bit-exact where every partial sum is exactly representable
(integer-valued inputs, reference known answers); otherwise
max|err| <= 1e-4 * sqrt(K) * max|a| * max|b| (the north-star GEMM bound).
"""
import numpy as np
import pytest

from _util import gemm_tol, rows_parallel, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _oracle():
    from oracle import oracle
    return oracle


def test_reference_known_answers(torch_dev):
    gh = _gh()
    # ghostflow-core/src/ops/matmul.rs:331-352
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(1, 7, dtype=np.float32).reshape(3, 2)
    c = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    assert c.tolist() == [[22.0, 28.0], [49.0, 64.0]]
    # ghostflow-core/tests/test_optimizations.rs:65-91
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    c = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    assert c.reshape(-1).tolist() == [19.0, 22.0, 43.0, 50.0]


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 3, 5), (33, 29, 17), (64, 64, 64), (128, 200, 96),
                                   (257, 300, 131), (1024, 1024, 1024), (1500, 300, 1300), (2048, 96, 2048),
                                   (300, 4100, 200), (130, 600, 70)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_integer_inputs_bit_exact(torch_dev, m, k, n, ta, tb):
    """|a|,|b| <= 8 integers: every partial sum < 2^24 is exact, so the GPU
    must equal the oracle bit for bit whatever the summation order.  The
    shapes cover all three tilings (64x64 below 128 tiles of 128x128,
    128x64 up to 512 of them, 128x128 beyond) with ragged edges, and long K
    on few tiles (300 x 4100 x 200)."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(m * 1000003 + k * 1009 + n)
    a = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
    b = rng.integers(-8, 9, size=(k, n)).astype(np.float32)
    ref = O.matmul(a, b)
    da = to_dev(a.T.copy() if ta else a, torch_dev)
    db = to_dev(b.T.copy() if tb else b, torch_dev)
    got = to_np(gh.sgemm(da, db, trans_a=bool(ta), trans_b=bool(tb)))
    np.testing.assert_array_equal(got, ref)


def test_config1_1024_normal(torch_dev):
    """Config 1: A, B [1024,1024] ~ N(0,1) from seed 0, full output vs oracle."""
    gh, O = _gh(), _oracle()
    a = gh.normal((1024, 1024), seed=0, tensor_id=0)
    b = gh.normal((1024, 1024), seed=0, tensor_id=1)
    ref = O.matmul(a, b)
    got = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    err = np.abs(got - ref).max()
    assert err <= gemm_tol(1024, a, b), err


@pytest.mark.parametrize("m,k,n", [(5, 7, 3), (100, 37, 130), (129, 64, 255)])
def test_unaligned_leading_dims(torch_dev, m, k, n):
    """Odd K / N: the scalar (non-16-byte) load path."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(7)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    assert np.abs(got - O.matmul(a, b)).max() <= gemm_tol(k, a, b)


@pytest.mark.parametrize("m,k,n", [(70, 96, 150), (70, 2048, 150)])
def test_alpha_beta_bias(torch_dev, m, k, n):
    """alpha, beta and bias: each a separate rounding after the sum."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(11)
    a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    b = rng.integers(-4, 5, size=(k, n)).astype(np.float32)
    c0 = rng.integers(-4, 5, size=(m, n)).astype(np.float32)
    bias = rng.integers(-4, 5, size=(n,)).astype(np.float32)
    dc = to_dev(c0, torch_dev)
    gh.sgemm(to_dev(a, torch_dev), to_dev(b, torch_dev), alpha=2.0, beta=-1.0, bias=to_dev(bias, torch_dev), out=dc)
    ref = 2.0 * O.matmul(a, b) - c0 + bias
    np.testing.assert_array_equal(to_np(dc), ref.astype(np.float32))


def test_beta_zero_ignores_nan_output(torch_dev):
    """beta == 0 must not read C (NaN in C stays out of the result)."""
    import torch
    gh = _gh()
    a = np.ones((40, 8), np.float32)
    b = np.ones((8, 50), np.float32)
    out = torch.full((40, 50), float("nan"), device=torch_dev)
    gh.sgemm(to_dev(a, torch_dev), to_dev(b, torch_dev), out=out)
    assert (to_np(out) == 8.0).all()


@pytest.mark.parametrize("m,n,k,tb", [(4096, 4096, 32, True), (2048, 2048, 32, False), (2100, 2000, 32, True),
                                      (512, 512, 64, False), (16, 4096, 256, True), (2, 1000, 512, True)])
def test_beta_zero_ignores_nan_output_every_path(torch_dev, m, n, k, tb):
    """The same contract on every kernel gfh_sgemm routes to: 256 x 256,
    128 x 128 with 3 and 2 ring stages, 64 x 64 (direct-to-LDS tiles), the
    skinny MFMA kernel (16 rows) and the row-dot GEMV (2 rows), with a bias;
    integer data, so the result is exact."""
    import torch
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    w = rng.integers(-4, 5, size=(n, k)).astype(np.float32)
    bias = rng.integers(-4, 5, size=(n,)).astype(np.float32)
    out = torch.full((m, n), float("nan"), device=torch_dev)
    b_dev = to_dev(w if tb else np.ascontiguousarray(w.T), torch_dev)
    gh.sgemm(to_dev(a, torch_dev), b_dev, trans_b=tb, bias=to_dev(bias, torch_dev), out=out)
    np.testing.assert_array_equal(to_np(out), (O.linear_forward(a, w) + bias).astype(np.float32))


def test_linear_known_small(torch_dev):
    """Linear::forward restated: x W^T + b, integer data -> exact."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(3)
    x = rng.integers(-5, 6, size=(16, 64)).astype(np.float32)
    w = rng.integers(-5, 6, size=(48, 64)).astype(np.float32)
    bias = rng.integers(-5, 6, size=(48,)).astype(np.float32)
    got = to_np(gh.linear(to_dev(x, torch_dev), to_dev(w, torch_dev), to_dev(bias, torch_dev)))
    np.testing.assert_array_equal(got, O.linear_forward(x, w, bias))


def test_config2_linear_4096_sampled_rows(torch_dev):
    """Config 2 at full size: x [4096,4096] ~ N(0,1), W, b ~ U(-1/64,1/64).
    Output rows are independent, so 256 sampled rows (plus the first and
    last) are checked against the oracle's Linear::forward on those rows."""
    gh, O = _gh(), _oracle()
    x = gh.normal((4096, 4096), seed=0, tensor_id=0)
    w = gh.uniform((4096, 4096), -1 / 64, 1 / 64, seed=0, tensor_id=1)
    bias = gh.uniform((4096,), -1 / 64, 1 / 64, seed=0, tensor_id=2)
    y = to_np(gh.linear(to_dev(x, torch_dev), to_dev(w, torch_dev), to_dev(bias, torch_dev)))
    rows = np.random.default_rng(0).choice(np.arange(1, 4095), 256, replace=False)
    rows = np.concatenate([[0, 4095], rows])
    ref = rows_parallel(O.linear_forward, x[rows], w, bias)
    err = np.abs(y[rows] - ref).max()
    assert err <= gemm_tol(4096, x, w), err


def test_batched_modulo_semantics(torch_dev):
    """batched_matmul takes batch slices modulo each operand's batch count
    (matmul.rs:148-149): [2,3,m,k] @ [3,k,n] broadcasts B over dim 0."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(5)
    a = rng.integers(-6, 7, size=(2, 3, 20, 24)).astype(np.float32)
    b = rng.integers(-6, 7, size=(3, 24, 36)).astype(np.float32)
    got = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    ref = O.batched_matmul(a, b)
    assert got.shape == (2, 3, 20, 36)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("n", [2048, 4096, 8192])
def test_square_sweep_sampled_rows(torch_dev, n):
    """The config-2 square sweep, A, B [n, n] ~ N(0,1) from seed 0 through
    Tensor::matmul (NN): 256 sampled rows of C (plus the first and last)
    against the oracle's matmul_blocked, within the GEMM bound.  Rows of C
    are independent, so a row subset is checked exactly as the full C."""
    gh, O = _gh(), _oracle()
    a = gh.normal((n, n), seed=0, tensor_id=0)
    b = gh.normal((n, n), seed=0, tensor_id=1)
    c = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    rows = np.random.default_rng(1).choice(np.arange(1, n - 1), 256, replace=False)
    rows = np.concatenate([[0, n - 1], rows])
    ref = rows_parallel(O.matmul, a[rows], b)
    err = np.abs(c[rows] - ref).max()
    assert err <= gemm_tol(n, a, b), err


def test_k_zero_gives_bias(torch_dev):
    import torch
    gh = _gh()
    a = torch.empty((4, 0), device=torch_dev)
    b = torch.empty((0, 6), device=torch_dev)
    bias = torch.arange(6, dtype=torch.float32, device=torch_dev)
    out = gh.sgemm(a, b, bias=bias)
    assert to_np(out).tolist() == [list(range(6))] * 4


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 256), (4100, 4000, 288), (4352, 3900, 32), (2048, 2048, 64),
                                   (2100, 2000, 96), (1024, 4096, 32), (330, 700, 96), (1000, 520, 1024),
                                   (1024, 1024, 1024)])
@pytest.mark.parametrize("tb", [True, False])
@pytest.mark.parametrize("ta", [False, True])
def test_big_tiles_integer_exact(torch_dev, m, n, k, tb, ta):
    """The four layouts with K % 32 == 0 (B as Linear's [n, k] weight or
    Tensor::matmul's [k, n]; A as [m, k] or, transposed as matmul_backward's
    a^T, [k, m]) take the direct-to-LDS kernel: 256 x 256 tiles (the first
    two: K >= 256), 128 x 128 tiles with 2 stages (4352 x 3900, 2100 x 2000)
    or a 3-deep ring (one round of tiles: 2048^2, 1024 x 4096), and 64 x 64
    tiles on 2 x 2 waves (the last three) -- ragged m and n inside the last
    tiles, alpha, beta and bias, on integer data (exact in any summation
    order).  The reference is the oracle's Linear::forward, or for the
    largest products the same sums in float64, which are exact here."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    w = rng.integers(-4, 5, size=(n, k)).astype(np.float32)
    c0 = rng.integers(-4, 5, size=(m, n)).astype(np.float32)
    bias = rng.integers(-4, 5, size=(n,)).astype(np.float32)
    dc = to_dev(c0, torch_dev)
    a_dev = to_dev(np.ascontiguousarray(a.T) if ta else a, torch_dev)
    b_dev = to_dev(w if tb else np.ascontiguousarray(w.T), torch_dev)
    gh.sgemm(a_dev, b_dev, trans_a=ta, trans_b=tb, alpha=2.0, beta=-1.0, bias=to_dev(bias, torch_dev), out=dc)
    if m * n * k <= (1 << 30):
        prod = O.linear_forward(a, w)
    else:
        prod = (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    ref = (2.0 * prod - c0 + bias).astype(np.float32)
    np.testing.assert_array_equal(to_np(dc), ref)


@pytest.mark.parametrize("m,n,k", [(32, 4096, 4096), (48, 1000, 2048), (64, 512, 4096), (100, 700, 3072),
                                   (17, 4100, 1024), (128, 4096, 2048), (768, 760, 2048), (384, 11000, 1024),
                                   (24, 11008, 2048)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_big_tiles_split_k_integer_exact(torch_dev, m, n, k, ta, tb):
    """Launches that split K over the CUs (2-8 slices whose partial tiles the
    last slice to arrive sums in slice order): fewer than 256 tiles of 64 x
    64 (32 x 64 up to 32 rows: 17, 24 and 32 rows here), 128 x 128 tiles
    where those fill more CUs (768 x 760), and 128 x 128 tiles two per CU
    that fill a partial round (384 x 11000: 258 tiles in 4 slices); ragged m
    and n, alpha, beta and bias, on integer data (exact in any order); the
    same call twice, so the arrival counters are back at zero."""
    gh = _gh()
    rng = np.random.default_rng(m + 3 * n + k + 5 * ta + tb)
    if ta and m % 4:
        pytest.skip("a transposed A takes the tile kernels with m % 4 == 0")
    a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    w = rng.integers(-4, 5, size=(n, k)).astype(np.float32)
    c0 = rng.integers(-4, 5, size=(m, n)).astype(np.float32)
    bias = rng.integers(-4, 5, size=(n,)).astype(np.float32)
    a_dev = to_dev(np.ascontiguousarray(a.T) if ta else a, torch_dev)
    b_dev = to_dev(w if tb else np.ascontiguousarray(w.T), torch_dev)
    ref = (2.0 * (a.astype(np.float64) @ w.astype(np.float64).T) - c0 + bias).astype(np.float32)
    for _ in range(2):
        dc = to_dev(c0, torch_dev)
        gh.sgemm(a_dev, b_dev, trans_a=bool(ta), trans_b=bool(tb), alpha=2.0, beta=-1.0, bias=to_dev(bias, torch_dev),
                 out=dc)
        np.testing.assert_array_equal(to_np(dc), ref)


@pytest.mark.parametrize("m,n,k", [(32, 4096, 4096), (64, 512, 4096)])
def test_big_tiles_split_k_random(torch_dev, m, n, k):
    """Split K on N(0, 1) data against the oracle's matmul_blocked, within
    the GEMM bound, and bit-identical on a second call (the slices are
    summed in a fixed order whatever order they arrive in)."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(m + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    da, db = to_dev(a, torch_dev), to_dev(b, torch_dev)
    got = to_np(gh.sgemm(da, db))
    assert np.abs(got - O.matmul(a, b)).max() <= gemm_tol(k, a, b)
    np.testing.assert_array_equal(to_np(gh.sgemm(da, db)), got)


def _strided_batched(torch_dev, ta, tb, a, b, batch_a, batch_b, batch, m, n, k, alpha=1.0, beta=0.0, c0=None,
                     bias=None):
    """gfh_sgemm_strided_batched on packed slices; returns C [batch, m, n]
    (C starts as c0, or NaN when beta is 0)."""
    import torch
    gh = _gh()
    L = gh.lib()
    da, db = to_dev(a, torch_dev), to_dev(b, torch_dev)
    dc = to_dev(c0, torch_dev) if c0 is not None else torch.full((batch, m, n), float("nan"), device=torch_dev)
    dbias = to_dev(bias, torch_dev) if bias is not None else None
    st = torch.cuda.current_stream(torch_dev).cuda_stream
    rc = L.gfh_sgemm_strided_batched(int(ta), int(tb), m, n, k, alpha, da.data_ptr(), m if ta else k, m * k, batch_a,
                                     db.data_ptr(), k if tb else n, k * n, batch_b, beta, dc.data_ptr(), n, m * n,
                                     batch, None if dbias is None else dbias.data_ptr(), st)
    assert rc == 0, L.gfh_last_error()
    return to_np(dc)


@pytest.mark.parametrize("batch,batch_a,batch_b,m,n,k", [
    (4, 4, 1, 2048, 2048, 256),   # 256 x 256 tiles, B shared by every slice
    (16, 16, 16, 512, 512, 128),  # 128 x 128 tiles, one round (3-deep ring), the SDPA score shape
    (32, 32, 32, 512, 512, 96),   # 128 x 128 tiles, 2 stages
    (6, 3, 6, 256, 320, 96),      # 64 x 64 tiles, A slices taken modulo 3
    (6, 6, 3, 300, 260, 64),      # 64 x 64 tiles, B slices modulo 3, ragged edges
])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_big_tiles_batched_modulo(torch_dev, batch, batch_a, batch_b, m, n, k, ta, tb):
    """Strided-batched products: slice z multiplies A slice z % batch_a by B
    slice z % batch_b (batched_matmul's modulo indexing, matmul.rs:148-149),
    on integer data (exact in any order), plain and with alpha, beta and
    bias.  With A as [m, k] they run on the
    direct-to-LDS kernel, the batch as its grid's y dimension; a transposed
    A takes the general tile kernel."""
    rng = np.random.default_rng(batch * 7 + m + n + k + 3 * ta + tb)
    a = rng.integers(-4, 5, size=(batch_a, m, k)).astype(np.float32)
    b = rng.integers(-4, 5, size=(batch_b, k, n)).astype(np.float32)
    a_st = np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a
    b_st = np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b
    got = _strided_batched(torch_dev, ta, tb, a_st, b_st, batch_a, batch_b, batch, m, n, k)
    for z in range(batch):
        ref = (a[z % batch_a].astype(np.float64) @ b[z % batch_b].astype(np.float64)).astype(np.float32)
        np.testing.assert_array_equal(got[z], ref, err_msg=f"slice {z}")
    # alpha, beta (each slice's own C) and bias, separately rounded
    c0 = rng.integers(-4, 5, size=(batch, m, n)).astype(np.float32)
    bias = rng.integers(-4, 5, size=(n,)).astype(np.float32)
    got = _strided_batched(torch_dev, ta, tb, a_st, b_st, batch_a, batch_b, batch, m, n, k, alpha=2.0, beta=-1.0,
                           c0=c0, bias=bias)
    for z in range(batch):
        prod = (a[z % batch_a].astype(np.float64) @ b[z % batch_b].astype(np.float64)).astype(np.float32)
        np.testing.assert_array_equal(got[z], (2.0 * prod - c0[z] + bias).astype(np.float32), err_msg=f"slice {z}")


@pytest.mark.parametrize("m", [1, 3, 8, 13, 16])
def test_matmul_decode_rows(torch_dev, m):
    """Tensor::matmul at decode batch sizes (x [m, k] . W [k, n], m <= 16)
    runs on the decode GEMV kernel: bit-exact on integer data, and within
    the GEMM bound on N(0, 1) data against the oracle's matmul_blocked."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(40 + m)
    k, n = 1000, 4100
    a = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
    b = rng.integers(-8, 9, size=(k, n)).astype(np.float32)
    np.testing.assert_array_equal(to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev))), O.matmul(a, b))
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    assert np.abs(got - O.matmul(a, b)).max() <= gemm_tol(k, a, b)


@pytest.mark.parametrize("n", [2048, 4096])
def test_big_tiles_nn_random(torch_dev, n):
    """NN at n^3 on N(0,1) data (the sweep's shapes: 128 x 128 tiles at 2048,
    256 x 256 at 4096) against the oracle on sampled rows, within the GEMM
    bound."""
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(8)
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    got = to_np(gh.sgemm(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    rows = rng.choice(n, size=256, replace=False)
    ref = rows_parallel(O.matmul, a[rows], b)
    assert np.abs(got[rows] - ref).max() <= gemm_tol(n, a, b)


@pytest.mark.parametrize("m,n", [(4096, 4096), (1000, 900)])
def test_nt_big_tiles_strided(torch_dev, m, n):
    """lda > k and ldc > n on the 256 x 256 and the 64 x 64 kernels; bytes
    between rows of C stay untouched."""
    import torch
    gh, O = _gh(), _oracle()
    rng = np.random.default_rng(31)
    k, lda, ldc = 96, 100, n + 4
    xa = rng.integers(-4, 5, size=(m, lda)).astype(np.float32)
    w = rng.integers(-4, 5, size=(n, k)).astype(np.float32)
    dx, dw = to_dev(xa, torch_dev), to_dev(w, torch_dev)
    out = torch.full((m, ldc), 7.0, device=torch_dev)
    rc = gh.lib().gfh_sgemm(0, 1, m, n, k, 1.0, dx.data_ptr(), lda, dw.data_ptr(), k, 0.0, out.data_ptr(), ldc,
                            None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    got = to_np(out)
    np.testing.assert_array_equal(got[:, :n], O.linear_forward(np.ascontiguousarray(xa[:, :k]), w))
    assert (got[:, n:] == 7.0).all()
