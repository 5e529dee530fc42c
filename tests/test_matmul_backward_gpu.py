"""GPU parity of matmul_backward (ghostflow-autograd/src/backward.rs:131-160):
grad_a = grad . b^T and grad_b = a^T . grad through gfh_matmul_backward_f32
(an NT and a TN gfh_sgemm).  Bars: bit-exact on integer-valued inputs (every
partial sum exact in any order), otherwise the fp32 GEMM bound with K = n
for grad_a and K = m for grad_b."""
import numpy as np
import pytest

from oracle import oracle as O
from _util import gemm_tol, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


# decode-size rows (GEMV / skinny NT), tile sizes, ragged edges, K = 1
@pytest.mark.parametrize("m,k,n", [(1, 64, 96), (3, 100, 257), (16, 256, 130), (64, 33, 70), (130, 257, 1),
                                   (512, 384, 256), (1000, 40, 1100)])
def test_matmul_backward_integer_exact(torch_dev, m, k, n):
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    g, a, b = (rng.integers(-8, 9, size=s).astype(np.float32) for s in ((m, n), (m, k), (k, n)))
    ga, gb = _gh().matmul_backward(to_dev(g, torch_dev), to_dev(a, torch_dev), to_dev(b, torch_dev))
    ra, rb = O.matmul_backward(g, a, b)
    np.testing.assert_array_equal(to_np(ga), ra)
    np.testing.assert_array_equal(to_np(gb), rb)


@pytest.mark.parametrize("m,k,n", [(4096, 1024, 1024), (8, 4096, 4096), (1024, 4096, 4096)])
def test_matmul_backward_random(torch_dev, m, k, n):
    rng = np.random.default_rng(m + k + n)
    g, a, b = (rng.standard_normal(s).astype(np.float32) for s in ((m, n), (m, k), (k, n)))
    ga, gb = _gh().matmul_backward(to_dev(g, torch_dev), to_dev(a, torch_dev), to_dev(b, torch_dev))
    ga, gb = to_np(ga), to_np(gb)
    # rows of grad_a and rows of grad_b are independent: check a sample of each
    ri = rng.choice(m, size=min(m, 64), replace=False)
    rj = rng.choice(k, size=min(k, 64), replace=False)
    ra, _ = O.matmul_backward(g[ri], a[ri], b)
    _, rb = O.matmul_backward(g, a[:, rj], b[rj])
    assert np.abs(ga[ri] - ra).max() <= gemm_tol(n, g, b)
    assert np.abs(gb[rj] - rb).max() <= gemm_tol(m, a, g)


def test_matmul_backward_one_side(torch_dev):
    rng = np.random.default_rng(9)
    g, a, b = (rng.integers(-4, 5, size=s).astype(np.float32) for s in ((20, 30), (20, 10), (10, 30)))
    gh = _gh()
    ga, gb = gh.matmul_backward(to_dev(g, torch_dev), to_dev(a, torch_dev), to_dev(b, torch_dev), need_b=False)
    assert gb is None
    np.testing.assert_array_equal(to_np(ga), O.matmul_backward(g, a, b)[0])
    ga, gb = gh.matmul_backward(to_dev(g, torch_dev), to_dev(a, torch_dev), to_dev(b, torch_dev), need_a=False)
    assert ga is None
    np.testing.assert_array_equal(to_np(gb), O.matmul_backward(g, a, b)[1])
