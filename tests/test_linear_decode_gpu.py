"""Linear::forward at decode sizes (x [m <= 64, k] . W^T, W [out, in]) on the
GPU: gfh_sgemm sends these NT calls to the row-dot GEMV kernel (m <= 4) or
to the skinny f32-MFMA kernel (4 < m <= 64).  Against
the oracle's Linear::forward / matmul (ghostflow-nn/src/linear.rs:56-69,
ghostflow-core/src/ops/matmul.rs:91-170).  Bars: bit-exact on
integer-valued inputs (every partial sum exact in any order), otherwise the
north-star GEMM bound."""
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


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 17, 33, 48, 64])
@pytest.mark.parametrize("k,n", [(4, 1), (256, 17), (260, 300), (1000, 4100), (4100, 300), (4096, 16385)])
def test_nt_gemv_integer_exact(torch_dev, m, k, n):
    """GEMV (m <= 4): k = 260 / 1000 end in a partial 256-element step; n =
    4100 / 16385 give the 2- and 4-row tilings a ragged last wave.  Skinny
    MFMA (m > 4): ragged m inside a 16-row block, ragged n inside a 16-column
    block, k % 16 != 0, and 4100 x 300 splits K over 4 workgroups (the last
    slice shorter)."""
    if m > 8 and n * k > 4096 * 4100:
        pytest.skip("oracle time; the large n is covered at m <= 8 and by test_decode_linear_4096")
    gh, O = _gh(), _O()
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    x = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
    w = rng.integers(-8, 9, size=(n, k)).astype(np.float32)
    bias = rng.integers(-8, 9, size=(n,)).astype(np.float32)
    got = to_np(gh.linear(to_dev(x, torch_dev), to_dev(w, torch_dev), to_dev(bias, torch_dev)))
    np.testing.assert_array_equal(got, O.linear_forward(x, w, bias))


@pytest.mark.parametrize("m,k,n", [(3, 520, 777), (6, 520, 777), (20, 4100, 100)])
def test_nt_gemv_alpha_beta(torch_dev, m, k, n):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(21)
    x = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    w = rng.integers(-4, 5, size=(n, k)).astype(np.float32)
    c0 = rng.integers(-4, 5, size=(m, n)).astype(np.float32)
    bias = rng.integers(-4, 5, size=(n,)).astype(np.float32)
    dc = to_dev(c0, torch_dev)
    gh.sgemm(to_dev(x, torch_dev), to_dev(w, torch_dev), trans_b=True, alpha=2.0, beta=-1.0,
             bias=to_dev(bias, torch_dev), out=dc)
    ref = 2.0 * O.matmul(x, np.ascontiguousarray(w.T)) - c0 + bias
    np.testing.assert_array_equal(to_np(dc), ref.astype(np.float32))


@pytest.mark.parametrize("m", [4, 24])
def test_nt_gemv_strided_rows(torch_dev, m):
    """lda > k and ldc > n (rows of a larger buffer, as when a projection
    writes into a KV cache); the bytes between rows stay untouched."""
    import torch
    gh, O = _gh(), _O()
    rng = np.random.default_rng(22)
    k, n, lda, ldc = 512, 300, 520, 1000
    xa = rng.integers(-8, 9, size=(m, lda)).astype(np.float32)
    w = rng.integers(-8, 9, size=(n, k)).astype(np.float32)
    dx, dw = to_dev(xa, torch_dev), to_dev(w, torch_dev)
    out = torch.full((m, ldc), 7.0, device=torch_dev)
    rc = gh.lib().gfh_sgemm(0, 1, m, n, k, 1.0, dx.data_ptr(), lda, dw.data_ptr(), k, 0.0, out.data_ptr(), ldc,
                            None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    got = to_np(out)
    np.testing.assert_array_equal(got[:, :n], O.linear_forward(np.ascontiguousarray(xa[:, :k]), w))
    assert (got[:, n:] == 7.0).all()


@pytest.mark.parametrize("m", [2, 12])
def test_nt_gemv_batched_modulo(torch_dev, m):
    """Batched NT with one shared weight (batch_b = 1): every batch slice
    uses W, as the reference's modulo indexing gives (matmul.rs:148-149)."""
    import torch
    gh, O = _gh(), _O()
    rng = np.random.default_rng(23)
    batch, k, n = 3, 256, 129
    x = rng.integers(-8, 9, size=(batch, m, k)).astype(np.float32)
    w = rng.integers(-8, 9, size=(n, k)).astype(np.float32)
    dx, dw = to_dev(x, torch_dev), to_dev(w, torch_dev)
    out = torch.empty((batch, m, n), device=torch_dev)
    rc = gh.lib().gfh_sgemm_strided_batched(0, 1, m, n, k, 1.0, dx.data_ptr(), k, m * k, batch, dw.data_ptr(), k,
                                            0, 1, 0.0, out.data_ptr(), n, m * n, batch, None,
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    ref = np.stack([O.linear_forward(x[i], w) for i in range(batch)])
    np.testing.assert_array_equal(to_np(out), ref)


@pytest.mark.parametrize("m", [1, 4, 8, 16, 64])

def test_decode_linear_4096(torch_dev, m):
    """x [m, 4096] ~ N(0,1), W [4096, 4096] and b ~ U(-1/64, 1/64) (the
    config-2 layer at decode batch sizes), against the GEMM bound."""
    gh, O = _gh(), _O()
    x = gh.normal((m, 4096), seed=3, tensor_id=0)
    w = gh.uniform((4096, 4096), -1 / 64, 1 / 64, seed=0, tensor_id=1)
    bias = gh.uniform((4096,), -1 / 64, 1 / 64, seed=0, tensor_id=2)
    got = to_np(gh.linear(to_dev(x, torch_dev), to_dev(w, torch_dev), to_dev(bias, torch_dev)))
    ref = O.linear_forward(x, w, bias)
    assert np.abs(got - ref).max() <= gemm_tol(4096, x, w)


@pytest.mark.parametrize("m,k,n,tb", [(1, 300, 200, True), (3, 1000, 130, True), (4, 4096, 512, True),
                                      (16, 520, 300, True), (64, 1024, 260, True), (300, 256, 520, True),
                                      (2, 300, 200, False), (300, 256, 520, False)])
def test_epilogue_rounding_non_integer(torch_dev, m, k, n, tb):
    """alpha, beta and bias with non-integer values (0.7, -1.3, random
    bias): the epilogue is alpha * acc, then + beta * C, then + bias, each a
    separately rounded f32 operation -- no FMA -- on every route (row-dot
    GEMV at m <= 4, skinny MFMA, tiles).  Checked bit for bit against the
    same route run with alpha = 1, beta = 0 and no bias, rounded on the host
    in that order."""
    import torch
    gh = _gh()
    rng = np.random.default_rng(m * 13 + k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    dx = to_dev(x, torch_dev)
    dw = to_dev(w if tb else np.ascontiguousarray(w.T), torch_dev)
    acc = to_np(gh.sgemm(dx, dw, trans_b=tb))
    out = to_dev(c0, torch_dev)
    gh.sgemm(dx, dw, trans_b=tb, alpha=0.7, beta=-1.3, bias=to_dev(bias, torch_dev), out=out)
    a32, b32 = np.float32(0.7), np.float32(-1.3)
    ref = ((a32 * acc).astype(np.float32) + (b32 * c0).astype(np.float32)).astype(np.float32)
    ref = (ref + bias).astype(np.float32)
    np.testing.assert_array_equal(to_np(out).view(np.uint32), ref.view(np.uint32))
    torch.cuda.synchronize()
