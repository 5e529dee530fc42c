"""The Tensor-level C API (include/ghostflow.h) on the GPU against the
oracle: create/data round trips, zeros/ones, broadcast add/mul (bit-exact
against the restatement of broadcast_binary_op), matmul (2-D within the
GEMM bound, exact on integer data; batched with the reference's modulo batch
indexing), reshape sharing the buffer, and the reference's error codes."""
import ctypes as C

import numpy as np
import pytest

from _capi import COMPUTATION_FAILED, INVALID_SHAPE, SUCCESS, T, call2, create, dims, lib
from _util import gemm_tol

pytestmark = pytest.mark.gpu


def _O():
    from oracle import oracle
    return oracle


@pytest.fixture(autouse=True)
def _init(torch_dev):
    assert lib().ghostflow_init() == SUCCESS
    yield


@pytest.mark.parametrize("shape", [(3,), (2, 3), (4, 1, 5), (), (0, 3), (1000, 37)])
def test_create_data_round_trip(shape):
    a = np.random.default_rng(len(shape)).standard_normal(shape).astype(np.float32)
    t = create(a)
    assert t.shape() == shape
    np.testing.assert_array_equal(t.numpy(), a)


@pytest.mark.parametrize("name,value", [("zeros", 0.0), ("ones", 1.0)])
def test_zeros_ones(name, value):
    h = C.c_void_p()
    d, nd = dims((7, 1, 9))
    assert getattr(lib(), "ghostflow_tensor_" + name)(d, nd, C.byref(h)) == SUCCESS
    t = T(h.value)
    assert t.shape() == (7, 1, 9)
    assert (t.numpy() == value).all()


def test_reference_add_known_answers():
    """arithmetic.rs:257-271."""
    rc, c = call2("add", create([1, 2, 3]), create([4, 5, 6]))
    assert rc == SUCCESS and c.numpy().tolist() == [5, 7, 9]
    rc, c = call2("add", create(np.array([[1], [2], [3]], np.float32)), create(np.array([[10, 20]], np.float32)))
    assert rc == SUCCESS and c.shape() == (3, 2)


@pytest.mark.parametrize("sa,sb", [((4, 1, 3), (2, 3)), ((5,), ()), ((), (2, 2)), ((3, 1), (1, 4)),
                                   ((2, 3, 4), (3, 1)), ((1, 1, 7), (6, 1, 1)), ((2, 0, 3), (1, 3)),
                                   ((1025, 513), (1025, 513)), ((1, 3), (1, 3)), ((256, 4096), (4096,)),
                                   ((8, 1, 16, 1), (1, 5, 1, 3))])
@pytest.mark.parametrize("op", ["add", "mul"])
def test_broadcast_binary_bit_exact(sa, sb, op):
    O = _O()
    rng = np.random.default_rng(sum(sa) + 3 * sum(sb))
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    rc, c = call2(op, create(a), create(b))
    assert rc == SUCCESS, lib().ghostflow_get_last_error()
    want = O.broadcast_binary(a, b, op)
    assert c.shape() == want.shape
    np.testing.assert_array_equal(c.numpy(), want)


def test_broadcast_incompatible_is_computation_failed():
    rc, c = call2("add", create(np.zeros((2, 3))), create(np.zeros((4,))))
    assert rc == COMPUTATION_FAILED and c is None
    assert b"broadcast" in lib().ghostflow_get_last_error()


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (64, 64, 64), (300, 257, 129), (1024, 1024, 1024)])
def test_matmul_2d(m, k, n):
    O = _O()
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    rc, c = call2("matmul", create(a), create(b))
    assert rc == SUCCESS, lib().ghostflow_get_last_error()
    assert c.shape() == (m, n)
    assert np.abs(c.numpy() - O.matmul(a, b)).max() <= gemm_tol(k, a, b)


def test_matmul_integer_exact_and_reference_known_answer():
    O = _O()
    # matmul.rs:331-352: [[1,2,3],[4,5,6]] . [[1,2],[3,4],[5,6]] = [[22,28],[49,64]]
    rc, c = call2("matmul", create(np.array([[1, 2, 3], [4, 5, 6]], np.float32)),
                  create(np.array([[1, 2], [3, 4], [5, 6]], np.float32)))
    assert rc == SUCCESS and c.numpy().tolist() == [[22, 28], [49, 64]]
    rng = np.random.default_rng(5)
    a = rng.integers(-8, 9, (200, 300)).astype(np.float32)
    b = rng.integers(-8, 9, (300, 100)).astype(np.float32)
    rc, c = call2("matmul", create(a), create(b))
    np.testing.assert_array_equal(c.numpy(), O.matmul(a, b))


@pytest.mark.parametrize("sa,sb", [((2, 3, 8, 16), (16, 4)), ((4, 8, 16), (1, 16, 4)), ((2, 1, 8, 16), (3, 16, 4)),
                                   ((5, 32, 64), (5, 64, 48)), ((3, 8, 16), (16, 4))])
def test_matmul_batched_modulo_indexing(sa, sb):
    """matmul.rs:122-170: output batch i reads A slice i % (A's batch count)
    and B slice i % (B's); ((2,1) x (3)) broadcasts to 6 batches whose
    operands are NOT the broadcast pairs, as in the reference."""
    O = _O()
    rng = np.random.default_rng(len(sa) * 7 + sa[0])
    a = rng.integers(-4, 5, sa).astype(np.float32)
    b = rng.integers(-4, 5, sb).astype(np.float32)
    rc, c = call2("matmul", create(a), create(b))
    assert rc == SUCCESS, lib().ghostflow_get_last_error()
    want = O.batched_matmul(a, b)
    assert c.shape() == want.shape
    np.testing.assert_array_equal(c.numpy(), want)


def test_matmul_empty_k_gives_zeros():
    rc, c = call2("matmul", create(np.zeros((3, 0))), create(np.zeros((0, 4))))
    assert rc == SUCCESS
    assert c.shape() == (3, 4) and (c.numpy() == 0).all()


def test_matmul_errors_are_computation_failed():
    """lib.rs:296-301 maps every Tensor::matmul error to ComputationFailed."""
    for sa, sb in (((3,), (3, 2)), ((2, 3), (4, 2)), ((4, 2, 3), (2, 3, 5))):
        rc, c = call2("matmul", create(np.zeros(sa)), create(np.zeros(sb)))
        assert rc == COMPUTATION_FAILED and c is None, (sa, sb)


def test_reshape_shares_buffer_and_checks_count():
    a = np.arange(12, dtype=np.float32)
    t = create(a.reshape(2, 6))
    h = C.c_void_p()
    d, nd = dims((3, 4))
    assert lib().ghostflow_tensor_reshape(t.h, d, nd, C.byref(h)) == SUCCESS
    r = T(h.value)
    t.free()  # the reshaped handle keeps the buffer alive
    assert r.shape() == (3, 4)
    np.testing.assert_array_equal(r.numpy(), a.reshape(3, 4))
    d5, nd5 = dims((5,))
    h2 = C.c_void_p()
    assert lib().ghostflow_tensor_reshape(r.h, d5, nd5, C.byref(h2)) == INVALID_SHAPE
    assert h2.value is None


def test_last_error_clears_on_success():
    call2("add", create(np.zeros((2, 3))), create(np.zeros((4,))))
    assert lib().ghostflow_get_last_error() != b"No error"
    rc, _ = call2("add", create([1.0]), create([2.0]))
    assert rc == SUCCESS
    assert lib().ghostflow_get_last_error() == b"No error"
