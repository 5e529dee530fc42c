"""int8 quantization, INT8 linear and dequantization on the GPU against the
oracle (quantization.rs restated).  Codes, scales, zero points and int32
accumulators must be bit-exact; the fp32 output of the INT8 linear must equal
the oracle's epilogue bit for bit and stay within the GEMM bound of the
reference's executable composite (dequantize both operands, fp32 matmul)."""
import numpy as np
import pytest

from _util import gemm_tol, rows_parallel, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _O():
    from oracle import oracle
    return oracle


def _same_f32(a, b):
    """Bitwise equality of float32 arrays (NaN-aware)."""
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


REF_INPUTS = [
    # (data, shape, per_channel, symmetric): the reference's own test inputs
    # (ghostflow-nn/src/quantization.rs:300-428)
    ([1, 2, 3, 4, 5, 6], (2, 3), False, True),
    ([1, 2, 3, 10, 20, 30], (2, 3), True, True),
    ([-5, -3, -1, 1, 3, 5], (6,), False, False),
    ([0.5, 1.5, 2.5], (3,), False, False),
    ([1, 2, 3, 4], (4,), True, True),
    ([1, 2, 3, 4], (2, 2), True, True),
]


@pytest.mark.parametrize("data,shape,per_channel,symmetric", REF_INPUTS)
def test_reference_inputs_bit_exact(torch_dev, data, shape, per_channel, symmetric):
    gh, O = _gh(), _O()
    x = np.array(data, np.float32).reshape(shape)
    if per_channel:
        q, s, z = gh.quantize_per_channel(to_dev(x, torch_dev), symmetric)
        rq, rs, rz = O.quantize_per_channel(x, symmetric)
    else:
        q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), symmetric)
        rq, rs, rz = O.quantize_per_tensor(x, symmetric)
    np.testing.assert_array_equal(to_np(q), rq)
    assert _same_f32(to_np(s).reshape(-1), np.atleast_1d(rs))
    np.testing.assert_array_equal(to_np(z).reshape(-1), np.atleast_1d(rz))
    deq = to_np(gh.dequantize(q, s, z))
    assert _same_f32(deq, O.dequantize(rq, rs, rz))


def test_hand_derived_codes(torch_dev):
    """Exact values worked out by hand from quantization.rs:77-108 (the
    asymmetric case is a half-away-from-zero tie: zp = round(-0.5) = -1)."""
    gh = _gh()
    x = np.array([-5, -3, -1, 1, 3, 5], np.float32)
    q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), False)
    assert to_np(q).tolist() == [-128, -78, -27, 25, 76, 126]
    assert int(to_np(z)[0]) == -1
    x = np.array([0.5, 1.5, 2.5], np.float32)
    q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), False)
    assert to_np(q).tolist() == [-64, 63, 127]
    assert int(to_np(z)[0]) == -128


@pytest.mark.parametrize("rows,cols", [(1, 1), (37, 129), (64, 4096), (11008, 4096)])
@pytest.mark.parametrize("symmetric", [True, False])
def test_per_channel_random(torch_dev, rows, cols, symmetric):
    gh, O = _gh(), _O()
    x = gh.normal((rows, cols), 0.0, 0.02, seed=0, tensor_id=1)
    q, s, z = gh.quantize_per_channel(to_dev(x, torch_dev), symmetric)
    rq, rs, rz = O.quantize_per_channel(x, symmetric)
    np.testing.assert_array_equal(to_np(q), rq)
    assert _same_f32(to_np(s), rs)
    np.testing.assert_array_equal(to_np(z), rz)


@pytest.mark.parametrize("n", [1, 5, 1000, 4096 * 256 + 3, 4096 * 4096])
@pytest.mark.parametrize("symmetric", [True, False])
def test_per_tensor_random(torch_dev, n, symmetric):
    gh, O = _gh(), _O()
    x = gh.normal((n,), seed=0, tensor_id=0)
    q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), symmetric)
    rq, rs, rz = O.quantize_per_tensor(x, symmetric)
    np.testing.assert_array_equal(to_np(q), rq)
    assert _same_f32(to_np(s), np.atleast_1d(rs))
    assert int(to_np(z)[0]) == int(rz)


# Sizes around the one-launch form for small tensors (up to 16 workgroups of
# 1024 threads, one float4 each, so 4096 <= n <= 65536) and its edges: a
# single workgroup, a last workgroup with a ragged share or a partial
# float4, and the sizes just outside its range (two launches).
ONE_LAUNCH_SIZES = [4095, 4096, 4097, 16384, 40000 + 3, 65533, 65536, 65537]


@pytest.mark.parametrize("n", ONE_LAUNCH_SIZES)
def test_per_tensor_one_launch_sizes(torch_dev, n):
    gh, O = _gh(), _O()
    x = gh.normal((n,), seed=5, tensor_id=0)
    for symmetric in (False, True):
        q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), symmetric)
        rq, rs, rz = O.quantize_per_tensor(x, symmetric)
        np.testing.assert_array_equal(to_np(q), rq)
        assert _same_f32(to_np(s), np.atleast_1d(rs))
        assert int(to_np(z)[0]) == int(rz)


def test_per_tensor_consecutive_calls(torch_dev):
    """Calls in a row on one stream with different sizes and data: each
    launch must see only its own workgroups' (min, max) pairs, so the
    arrival counters are back at zero after every call."""
    gh, O = _gh(), _O()
    for i, n in enumerate([65536, 4097, (1 << 20) + 1, 16384, 4096, 65533, 40003]):
        x = gh.normal((n,), 0.0, 1.0 + i, seed=40 + i, tensor_id=0)
        q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), False)
        rq, rs, rz = O.quantize_per_tensor(x, False)
        np.testing.assert_array_equal(to_np(q), rq, err_msg=str(n))
        assert _same_f32(to_np(s), np.atleast_1d(rs)), n
        assert int(to_np(z)[0]) == int(rz), n


@pytest.mark.parametrize("n", [4097, 16384, 65533])
def test_per_tensor_workgroups_that_stop_waiting(torch_dev, n, monkeypatch):
    """With a wait limit of 0 every workgroup of the one-launch form gives up
    waiting for the others and folds all of x itself: the same codes."""
    gh, O = _gh(), _O()
    monkeypatch.setenv("GFH_QUANT_WAIT_ROUNDS", "0")
    x = gh.normal((n,), seed=9, tensor_id=0)
    x[n // 3] = 40.0
    x[-1] = -35.0
    for symmetric in (False, True):
        q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), symmetric)
        rq, rs, rz = O.quantize_per_tensor(x, symmetric)
        np.testing.assert_array_equal(to_np(q), rq)
        assert _same_f32(to_np(s), np.atleast_1d(rs))
        assert int(to_np(z)[0]) == int(rz)
    monkeypatch.delenv("GFH_QUANT_WAIT_ROUNDS")
    q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), False)
    rq, rs, rz = O.quantize_per_tensor(x, False)
    np.testing.assert_array_equal(to_np(q), rq)


def test_special_values_one_launch(torch_dev):
    """The special-value patterns at sizes the one-launch form serves, with
    the extreme values in different workgroups and in the ragged tail."""
    gh, O = _gh(), _O()
    n = 65533
    base = gh.normal((n,), seed=12, tensor_id=0)
    cases = {"zeros": np.zeros(n, np.float32), "nan_only": np.full(n, np.nan, np.float32)}
    x = base.copy(); x[::797] = np.nan; cases["nans"] = x
    x = base.copy(); x[12347] = np.inf; cases["inf"] = x
    x = base.copy(); x[-1] = -np.inf; cases["neg_inf_in_tail"] = x
    x = base.copy(); x[-2] = 1e30; x[5] = -1e30; cases["huge"] = x
    cases["constant"] = np.full(n, -3.0, np.float32)
    for name, x in cases.items():
        for sym in (True, False):
            q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), sym)
            rq, rs, rz = O.quantize_per_tensor(x, sym)
            np.testing.assert_array_equal(to_np(q), rq, err_msg=f"{name} sym={sym}")
            assert _same_f32(to_np(s), np.atleast_1d(rs)), (name, sym)
            assert int(to_np(z)[0]) == int(rz), (name, sym)


def test_per_tensor_unaligned_view(torch_dev):
    """An offset (non 16-byte aligned) input takes the scalar path."""
    gh, O = _gh(), _O()
    base = gh.normal((1001,), seed=3, tensor_id=0)
    d = to_dev(base, torch_dev)[1:]
    q, s, z = gh.quantize_per_tensor(d, False)
    rq, rs, rz = O.quantize_per_tensor(base[1:], False)
    np.testing.assert_array_equal(to_np(q), rq)
    assert _same_f32(to_np(s), np.atleast_1d(rs))


def test_special_values(torch_dev):
    """NaN is ignored by the min/max folds and quantizes to zp; all-zero
    input gives scale 0 and code 0 (0/0 = NaN -> 0); infinities saturate."""
    gh, O = _gh(), _O()
    for data in ([0.0, 0.0, 0.0, 0.0], [1.0, np.nan, -2.0, 3.0], [np.inf, 1.0, -1.0, 2.0],
                 [-np.inf, 1.0, 0.5, 0.25], [7.0, 7.0, 7.0, 7.0], [-3.0, -3.0, -3.0, -3.0]):
        x = np.array(data, np.float32)
        for sym in (True, False):
            q, s, z = gh.quantize_per_tensor(to_dev(x, torch_dev), sym)
            rq, rs, rz = O.quantize_per_tensor(x, sym)
            np.testing.assert_array_equal(to_np(q), rq, err_msg=f"{data} sym={sym}")
            assert _same_f32(to_np(s), np.atleast_1d(rs)), (data, sym)
            assert int(to_np(z)[0]) == int(rz), (data, sym)
            qc, sc, zc = gh.quantize_per_channel(to_dev(x.reshape(2, 2), torch_dev), sym)
            rqc, rsc, rzc = O.quantize_per_channel(x.reshape(2, 2), sym)
            np.testing.assert_array_equal(to_np(qc), rqc)
            assert _same_f32(to_np(sc), rsc)


def test_dequantize_per_channel_large(torch_dev):
    gh, O = _gh(), _O()
    w = gh.normal((512, 1000), 0.0, 0.02, seed=0, tensor_id=1)
    rq, rs, rz = O.quantize_per_channel(w, False)
    got = to_np(gh.dequantize(to_dev(rq, torch_dev), to_dev(rs, torch_dev), to_dev(rz, torch_dev)))
    assert _same_f32(got, O.dequantize(rq, rs, rz))


def test_qweight_rowsum(torch_dev):
    gh = _gh()
    rng = np.random.default_rng(0)
    q = rng.integers(-128, 128, size=(300, 777)).astype(np.int8)
    got = to_np(gh.qweight_rowsum(to_dev(q, torch_dev)))
    np.testing.assert_array_equal(got, q.astype(np.int64).sum(1).astype(np.int32))


def _qlinear_case(torch_dev, m, n, k, x_per_row, with_zp, with_bias, seed=0):
    gh, O = _gh(), _O()
    x = gh.normal((m, k), seed=seed, tensor_id=0)
    w = gh.normal((n, k), 0.0, 0.02, seed=seed, tensor_id=1)
    bias = gh.uniform((n,), -1 / 64, 1 / 64, seed=seed, tensor_id=2) if with_bias else None
    qw, sw, _ = O.quantize_per_channel(w, True)
    if x_per_row:
        qx, sx, zx = O.quantize_per_channel(x, not with_zp)
    else:
        qx, sx, zx = O.quantize_per_tensor(x, not with_zp)
    zx_arg = np.atleast_1d(zx) if with_zp else None
    ry, racc = O.qlinear_i8(qx, sx, zx_arg, x_per_row, qw, sw, bias)
    d = lambda a: None if a is None else to_dev(np.ascontiguousarray(np.atleast_1d(a)), torch_dev)  # noqa: E731
    y, acc = gh.qlinear(d(qx), d(sx), d(zx_arg), d(qw), d(sw), x_per_row=x_per_row, bias=d(bias),
                        want_acc=True)
    np.testing.assert_array_equal(to_np(acc), racc)
    assert _same_f32(to_np(y), ry)
    # Within the GEMM bound of the reference composite: dequantize + matmul.
    dx = O.dequantize(qx.reshape(m, k), np.atleast_1d(sx), np.atleast_1d(zx))
    dw = O.dequantize(qw, sw, np.zeros(n, np.int8))
    comp = O.matmul(dx, O.transpose_last2(dw))
    if bias is not None:
        comp = comp + bias
    assert np.abs(to_np(y) - comp).max() <= gemm_tol(k, dx, dw) + 1e-6
    return x, w


@pytest.mark.parametrize("m,n,k", [(1, 48, 64), (5, 48, 64), (16, 1000, 256), (130, 257, 320), (256, 512, 4096)])
@pytest.mark.parametrize("x_per_row,with_zp", [(False, True), (True, False), (False, False)])
def test_qlinear_bit_exact(torch_dev, m, n, k, x_per_row, with_zp):
    _qlinear_case(torch_dev, m, n, k, x_per_row, with_zp, with_bias=(m % 2 == 1))


def test_qlinear_unaligned_k(torch_dev):
    """K not a multiple of 16: the byte-gather load path."""
    _qlinear_case(torch_dev, 33, 70, 77, False, True, True)


def test_qlinear_config3_w11008_sampled(torch_dev):
    """Config 3: W [11008,4096] ~ N(0,0.02) per-channel symmetric, x [M,4096]
    per-tensor asymmetric (DynamicQuantization::quantize_activation); int32
    accumulators of every row checked against an exact fp64 integer GEMM."""
    gh, O = _gh(), _O()
    n, k = 11008, 4096
    w = gh.normal((n, k), 0.0, 0.02, seed=0, tensor_id=1)
    dw = to_dev(w, torch_dev)
    qw, sw, zw = gh.quantize_per_channel(dw, True)
    rqw, rsw, _ = O.quantize_per_channel(w, True)
    np.testing.assert_array_equal(to_np(qw), rqw)
    for m in (1, 16, 256):
        x = gh.normal((m, k), seed=0, tensor_id=0)
        qx, sx, zx = gh.quantize_per_tensor(to_dev(x, torch_dev), False)
        rqx, rsx, rzx = O.quantize_per_tensor(x, False)
        np.testing.assert_array_equal(to_np(qx), rqx)
        y, acc = gh.qlinear(qx, sx, zx, qw, sw, want_acc=True)
        exact = (rqx.astype(np.float64) - float(rzx)) @ rqw.astype(np.float64).T
        np.testing.assert_array_equal(to_np(acc), exact.astype(np.int64).astype(np.int32))
        rows = np.arange(m) if m <= 16 else np.random.default_rng(m).choice(m, 16, replace=False)
        ry, _ = O.qlinear_i8(rqx[rows], rsx, np.atleast_1d(rzx), False, rqw, rsw)
        assert _same_f32(to_np(y)[rows], ry)


def test_qlinear_config3_m4096_w11008(torch_dev):
    """Config 3 at M = 4096, as the bench runs it: W [11008, 4096] ~
    N(0, 0.02) quantized per channel (symmetric), x [4096, 4096] ~ N(0, 1)
    quantized per tensor (asymmetric, DynamicQuantization::
    quantize_activation), the 256 x 256 tile kernel.  Every int32
    accumulator against the exact integer product (fp64 holds it exactly:
    |acc| < 2^31), and the output-only call (the bench's variant, no
    accumulator buffer) bit-exact to the oracle on 256 sampled rows plus the
    first and last."""
    gh, O = _gh(), _O()
    m, n, k = 4096, 11008, 4096
    w = gh.normal((n, k), 0.0, 0.02, seed=0, tensor_id=1)
    x = gh.normal((m, k), seed=0, tensor_id=0)
    qw, sw, _ = gh.quantize_per_channel(to_dev(w, torch_dev), True)
    qx, sx, zx = gh.quantize_per_tensor(to_dev(x, torch_dev), False)
    rqw, rsw, _ = O.quantize_per_channel(w, True)
    rqx, rsx, rzx = O.quantize_per_tensor(x, False)
    del w, x
    np.testing.assert_array_equal(to_np(qw), rqw)
    np.testing.assert_array_equal(to_np(qx), rqx)
    assert _same_f32(to_np(sx), np.atleast_1d(rsx)) and int(to_np(zx)[0]) == int(rzx)
    rowsum = gh.qweight_rowsum(qw)
    y_only, none = gh.qlinear(qx, sx, zx, qw, sw, w_rowsum=rowsum, want_acc=False)
    assert none is None
    _, acc = gh.qlinear(qx, sx, zx, qw, sw, w_rowsum=rowsum, want_y=False, want_acc=True)
    exact = (rqx.astype(np.float64) - float(rzx)) @ rqw.astype(np.float64).T
    np.testing.assert_array_equal(to_np(acc), exact.astype(np.int32))
    del exact, acc
    rows = np.random.default_rng(3).choice(np.arange(1, m - 1), 256, replace=False)
    rows = np.concatenate([[0, m - 1], rows])
    zxa = np.atleast_1d(rzx)
    ry = rows_parallel(lambda r: O.qlinear_i8(r, rsx, zxa, False, rqw, rsw, want_acc=False)[0], rqx[rows])
    assert _same_f32(to_np(y_only)[rows], ry)


def test_qlinear_4096_cube_sampled(torch_dev):
    """The 4096^3 int8 GEMM target shape: sampled rows of the int32
    accumulators against exact integer products."""
    gh, O = _gh(), _O()
    k = 4096
    x = gh.normal((4096, k), seed=0, tensor_id=0)
    w = gh.normal((4096, k), 0.0, 0.02, seed=0, tensor_id=1)
    qx, sx, zx = gh.quantize_per_channel(to_dev(x, torch_dev), True)
    qw, sw, _ = gh.quantize_per_channel(to_dev(w, torch_dev), True)
    y, acc = gh.qlinear(qx, sx, None, qw, sw, x_per_row=True, want_acc=True)
    rows = np.random.default_rng(4).choice(4096, 24, replace=False)
    hqx, hqw = to_np(qx), to_np(qw)
    exact = hqx[rows].astype(np.float64) @ hqw.astype(np.float64).T
    np.testing.assert_array_equal(to_np(acc)[rows], exact.astype(np.int32))
    ry, _ = O.qlinear_i8(hqx[rows], to_np(sx)[rows], None, True, hqw, to_np(sw))
    assert _same_f32(to_np(y)[rows], ry)


@pytest.mark.parametrize("m,n,k", [(1024, 256, 64), (1030, 300, 128), (1300, 777, 320), (2048, 384, 1024)])
@pytest.mark.parametrize("x_per_row,with_zp", [(False, True), (True, False), (True, True)])
def test_qlinear_large_tile_bit_exact(torch_dev, m, n, k, x_per_row, with_zp):
    """M >= 1024 with K % 64 == 0 takes the 256 x 256 tile kernel: ragged
    edge tiles in M and N, every activation-scale variant, int32
    accumulators and fp32 outputs bit-exact to the oracle."""
    _qlinear_case(torch_dev, m, n, k, x_per_row, with_zp, with_bias=(n % 2 == 1 or x_per_row))


@pytest.mark.parametrize("x_per_row", [False, True])
def test_qlinear_large_tile_y_only(torch_dev, x_per_row):
    """The output-only variant (no int32 accumulator buffer) of the large
    tile kernel equals the oracle bit for bit."""
    gh, O = _gh(), _O()
    m, n, k = 1280, 520, 256
    x = gh.normal((m, k), seed=9, tensor_id=0)
    w = gh.normal((n, k), 0.0, 0.02, seed=9, tensor_id=1)
    bias = gh.uniform((n,), -0.1, 0.1, seed=9, tensor_id=2)
    qw, sw, _ = O.quantize_per_channel(w, True)
    if x_per_row:
        qx, sx, zx = O.quantize_per_channel(x, False)
    else:
        qx, sx, zx = O.quantize_per_tensor(x, False)
    sx, zx = np.atleast_1d(sx), np.atleast_1d(zx)
    ry, _ = O.qlinear_i8(qx, sx, zx, x_per_row, qw, sw, bias)
    y, acc = gh.qlinear(to_dev(qx, torch_dev), to_dev(sx, torch_dev), to_dev(zx, torch_dev),
                        to_dev(qw, torch_dev), to_dev(sw, torch_dev), x_per_row=x_per_row,
                        bias=to_dev(bias, torch_dev), want_acc=False)
    assert acc is None
    assert _same_f32(to_np(y), ry)


@pytest.mark.parametrize("m,n,k", [(130, 257, 384), (192, 1100, 2048), (300, 4100, 1024), (500, 5000, 512)])
@pytest.mark.parametrize("x_per_row,with_zp", [(False, True), (True, False), (True, True)])
def test_qlinear_mid_m_tiles_bit_exact(torch_dev, m, n, k, x_per_row, with_zp):
    """64 < M <= 512 with K % 128 == 0 takes the largest tile that still
    gives ~160 workgroups: 64 x 64 (the first two shapes), 64 x 128 and
    128 x 128 -- ragged M and N on each, every activation-scale variant,
    int32 accumulators and fp32 outputs bit-exact to the oracle, through
    both the accumulator variant and the output-only one (whose LDS-staged
    stores take a single 32-row block per wave on the 64-row tiles)."""
    _qlinear_case(torch_dev, m, n, k, x_per_row, with_zp, with_bias=(n % 2 == 1))
    gh, O = _gh(), _O()
    x = gh.normal((m, k), seed=m, tensor_id=3)
    w = gh.normal((n, k), 0.0, 0.02, seed=m, tensor_id=4)
    bias = gh.uniform((n,), -0.1, 0.1, seed=m, tensor_id=5)
    qw, sw, _ = O.quantize_per_channel(w, True)
    if x_per_row:
        qx, sx, zx = O.quantize_per_channel(x, not with_zp)
    else:
        qx, sx, zx = O.quantize_per_tensor(x, not with_zp)
    sx, zx = np.atleast_1d(sx), np.atleast_1d(zx)
    zx_arg = zx if with_zp else None
    ry, _ = O.qlinear_i8(qx, sx, zx_arg, x_per_row, qw, sw, bias, want_acc=False)
    d = lambda a: None if a is None else to_dev(a, torch_dev)  # noqa: E731
    y, acc = gh.qlinear(d(qx), d(sx), d(zx_arg), d(qw), d(sw), x_per_row=x_per_row, bias=d(bias),
                        want_acc=False)
    assert acc is None
    assert _same_f32(to_np(y), ry)


def _qlinear_both_outputs(torch_dev, m, n, k, x_per_row, with_zp, seed):
    """y alone and (y, acc) from the GPU, each bit-exact to the oracle."""
    gh, O = _gh(), _O()
    x = gh.normal((m, k), seed=seed, tensor_id=0)
    w = gh.normal((n, k), 0.0, 0.02, seed=seed, tensor_id=1)
    bias = gh.uniform((n,), -0.1, 0.1, seed=seed, tensor_id=2)
    qw, sw, _ = O.quantize_per_channel(w, True)
    if x_per_row:
        qx, sx, zx = O.quantize_per_channel(x, not with_zp)
    else:
        qx, sx, zx = O.quantize_per_tensor(x, not with_zp)
    sx, zx = np.atleast_1d(sx), np.atleast_1d(zx)
    zx_arg = zx if with_zp else None
    ry, racc = O.qlinear_i8(qx, sx, zx_arg, x_per_row, qw, sw, bias)
    d = lambda a: None if a is None else to_dev(a, torch_dev)  # noqa: E731
    args = (d(qx), d(sx), d(zx_arg), d(qw), d(sw))
    y, acc = gh.qlinear(*args, x_per_row=x_per_row, bias=d(bias), want_acc=True)
    np.testing.assert_array_equal(to_np(acc), racc)
    assert _same_f32(to_np(y), ry)
    y2, _ = gh.qlinear(*args, x_per_row=x_per_row, bias=d(bias), want_acc=False)
    assert _same_f32(to_np(y2), ry)


@pytest.mark.parametrize("m,n,k", [(130, 1000, 8320), (250, 777, 10240), (200, 3000, 12288)])
@pytest.mark.parametrize("x_per_row,with_zp", [(False, True), (True, False), (True, True)])
def test_qlinear_split_k_bit_exact(torch_dev, m, n, k, x_per_row, with_zp):
    """64 < M <= 512 with K >= 8192 and few tiles splits K over workgroups
    (int32 partials, added by the last slice of each tile): 64 x 64 tiles in
    5 and 4 slices (the first two shapes), 128 x 128 in 5 with a shorter
    last slice (the third); ragged M and N, every activation-scale variant,
    both the accumulator output and the output-only path bit-exact."""
    _qlinear_both_outputs(torch_dev, m, n, k, x_per_row, with_zp, seed=m + k)


@pytest.mark.parametrize("m,k", [(128, 11008), (256, 11008), (256, 14336)])
def test_qlinear_split_k_swiglu_down(torch_dev, m, k):
    """The LLaMA / Mistral down projections at 128 and 256 rows (N = 4096):
    64 x 64 tiles in 2 slices at m = 128, 128 x 128 in 4 at m = 256 (the
    last one shorter at K = 11008, 86 stages); int32 accumulators and fp32
    outputs bit-exact."""
    _qlinear_both_outputs(torch_dev, m, 4096, k, False, True, seed=k)


@pytest.mark.parametrize("m,n,k", [(1, 1000, 4096), (7, 130, 1088), (16, 520, 2048), (17, 300, 4096),
                                   (33, 1000, 2048), (64, 130, 1088)])
@pytest.mark.parametrize("x_per_row,with_zp", [(False, True), (True, False), (True, True)])
def test_qlinear_skinny_bit_exact(torch_dev, m, n, k, x_per_row, with_zp):
    """M <= 64 with K % 16 == 0 streams the weight straight into i8 MFMA and
    splits K over workgroups (exact int32 partials, summed by the last
    workgroup of each column block): ragged N, 1-4 accumulator blocks,
    every activation-scale variant, bit-exact to the oracle."""
    _qlinear_case(torch_dev, m, n, k, x_per_row, with_zp, with_bias=(n % 2 == 0))


@pytest.mark.parametrize("m,n,k", [(1024, 128, 64), (1030, 300, 128), (1300, 777, 320), (2048, 384, 1024),
                                   (2304, 1152, 4096), (1024, 4096, 640)])
@pytest.mark.parametrize("x_per_row,with_zp", [(False, True), (True, False), (True, True)])
def test_qlinear_large_tile_y_variants_bit_exact(torch_dev, m, n, k, x_per_row, with_zp):
    """Output-only calls with M >= 1024 (the 256 x 256 tile kernel's
    LDS-staged output path): ragged edges, short and long K, every
    activation-scale variant -- fp32 outputs bit-exact to the oracle."""
    gh, O = _gh(), _O()
    x = gh.normal((m, k), seed=m + n, tensor_id=0)
    w = gh.normal((n, k), 0.0, 0.02, seed=m + n, tensor_id=1)
    bias = gh.uniform((n,), -0.1, 0.1, seed=m + n, tensor_id=2) if n % 2 == 0 else None
    qw, sw, _ = O.quantize_per_channel(w, True)
    if x_per_row:
        qx, sx, zx = O.quantize_per_channel(x, not with_zp)
    else:
        qx, sx, zx = O.quantize_per_tensor(x, not with_zp)
    sx, zx = np.atleast_1d(sx), np.atleast_1d(zx)
    zx_arg = zx if with_zp else None
    ry, _ = O.qlinear_i8(qx, sx, zx_arg, x_per_row, qw, sw, bias, want_acc=False)
    d = lambda a: None if a is None else to_dev(a, torch_dev)  # noqa: E731
    y, acc = gh.qlinear(d(qx), d(sx), d(zx_arg), d(qw), d(sw), x_per_row=x_per_row, bias=d(bias),
                        want_acc=False)
    assert acc is None
    assert _same_f32(to_np(y), ry)


@pytest.mark.parametrize("m,n,k", [(1, 1, 16), (1, 17, 80), (2, 100, 1040), (3, 33, 4096), (4, 1000, 4112),
                                   (1, 11008, 4096), (4, 4100, 11008)])
@pytest.mark.parametrize("x_per_row,with_zp", [(False, True), (True, False), (True, True)])
def test_qlinear_decode_rows_bit_exact(torch_dev, m, n, k, x_per_row, with_zp):
    """M <= 4 on the skinny kernel: k down to one 16-byte group, k % 64 != 0,
    ragged n inside a 16-column block, the config-3 weight at M = 1 and the
    SwiGLU down projection's K = 11008, every activation-scale variant,
    bit-exact to the oracle."""
    _qlinear_case(torch_dev, m, n, k, x_per_row, with_zp, with_bias=(n % 2 == 0))


def test_qlinear_decode_acc_only(torch_dev):
    """Accumulators without the fp32 output (sx / sw unused, NULL)."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(4)
    qx = rng.integers(-128, 128, size=(3, 2064), dtype=np.int8)
    qw = rng.integers(-127, 128, size=(70, 2064), dtype=np.int8)
    zx = np.array([-5], np.int8)
    _, racc = O.qlinear_i8(qx, np.ones(1, np.float32), zx, False, qw, np.ones(70, np.float32))
    y, acc = gh.qlinear(to_dev(qx, torch_dev), None, to_dev(zx, torch_dev), to_dev(qw, torch_dev), None,
                        want_y=False, want_acc=True)
    assert y is None
    np.testing.assert_array_equal(to_np(acc), racc)
