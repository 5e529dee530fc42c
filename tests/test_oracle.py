"""CPU tests that pin the oracle (oracle/gf_oracle.c) before it is trusted as
the checker of the HIP path.

Each check is one the reference itself holds (its unit-test known answers),
or one the mathematics fixes independently of the oracle's code: integer
inputs against an int64 brute force (exact in any order), fp64 brute force
with a rounding-error bound, closed forms (causal row 0, constant keys), and
hand-derived IEEE f32 values that a plausible mistake (round-half-even,
truncation, wrong operand order, dropped zero point) would change.
"""
import numpy as np
import pytest

from oracle import oracle as O

EPS = 2.0 ** -24


# ---------------------------------------------------------------------------
# GEMM: matmul_blocked (ghostflow-core/src/ops/matmul.rs:91-119)
# ---------------------------------------------------------------------------

def test_matmul_reference_known_answers():
    # matmul.rs:331-352
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(1, 7, dtype=np.float32).reshape(3, 2)
    assert O.matmul(a, b).tolist() == [[22.0, 28.0], [49.0, 64.0]]
    # ghostflow-core/tests/test_optimizations.rs:65-91
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    assert O.matmul(a, b).reshape(-1).tolist() == [19.0, 22.0, 43.0, 50.0]
    # Tensor::mv (matmul.rs:363-371) as a row-vector GEMM: [1,2] . [[1,3],[2,4]]
    x = np.array([[1, 2]], np.float32)
    wt = np.array([[1, 3], [2, 4]], np.float32)
    assert O.matmul(x, wt).tolist() == [[5.0, 11.0]]
    # dot = 32 (matmul.rs:354-361)
    assert O.matmul(np.array([[1, 2, 3]], np.float32),
                    np.array([[4], [5], [6]], np.float32)).item() == 32.0


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 5, 3), (33, 29, 17), (64, 200, 65), (3, 4096, 5)])
def test_matmul_integer_inputs_exact(m, k, n):
    rng = np.random.default_rng(m * 7 + k * 13 + n)
    a = rng.integers(-8, 9, size=(m, k))
    b = rng.integers(-8, 9, size=(k, n))
    got = O.matmul(a.astype(np.float32), b.astype(np.float32))
    np.testing.assert_array_equal(got, (a @ b).astype(np.float32))


def test_matmul_sums_k_sequentially():
    """Per element the reference adds products in ascending k, each add
    rounded: 2^24 + 1 + 1 -> 2^24 (each +1 is a tie that rounds to even),
    whereas any pairing of the ones first would give 2^24 + 2."""
    a = np.array([[2.0 ** 24, 1.0, 1.0]], np.float32)
    b = np.ones((3, 1), np.float32)
    assert O.matmul(a, b).item() == 2.0 ** 24
    a = np.array([[1.0, 1.0, 2.0 ** 24]], np.float32)
    assert O.matmul(a, b).item() == 2.0 ** 24 + 2
    # and it starts from +0.0: (-0.0) * 1 summed onto +0.0 gives +0.0
    z = O.matmul(np.array([[-0.0]], np.float32), np.array([[1.0]], np.float32)).item()
    assert z == 0.0 and np.copysign(1.0, z) == 1.0


def test_matmul_no_fma_contraction():
    """a*b + c with a*b inexact: separate roundings differ from an FMA.
    (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24; the product rounds to 1 + 2^-11
    (tie to even), so adding -(1 + 2^-11) yields exactly 0; an FMA would
    keep the 2^-24."""
    x = np.float32(1 + 2.0 ** -12)
    a = np.array([[x, 1.0]], np.float32)
    b = np.array([[x], [-(1 + 2.0 ** -11)]], np.float32)
    assert O.matmul(a, b).item() == 0.0


def test_matmul_fp64_error_bound():
    rng = np.random.default_rng(0)
    m, k, n = 37, 513, 41
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = O.matmul(a, b).astype(np.float64)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound = (k + 1) * EPS * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert (np.abs(got - exact) <= bound).all()


def test_matmul_identity_and_permutation():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((20, 20)).astype(np.float32)
    np.testing.assert_array_equal(O.matmul(a, np.eye(20, dtype=np.float32)), a)
    p = np.eye(20, dtype=np.float32)[rng.permutation(20)]
    np.testing.assert_array_equal(O.matmul(p, a), a[np.argmax(p, axis=1)])


def test_batched_matmul_modulo_indexing():
    """matmul.rs:147-149: output batch i uses A slice i % a_batch and B slice
    i % b_batch (flattened batch dims)."""
    rng = np.random.default_rng(2)
    a = rng.integers(-5, 6, size=(2, 3, 4, 6))
    b = rng.integers(-5, 6, size=(3, 6, 5))
    got = O.batched_matmul(a.astype(np.float32), b.astype(np.float32))
    assert got.shape == (2, 3, 4, 5)
    af = a.reshape(6, 4, 6)
    for i in range(6):
        np.testing.assert_array_equal(got.reshape(6, 4, 5)[i], (af[i] @ b[i % 3]).astype(np.float32))


def test_broadcast_binary_reference_known_answers():
    """arithmetic.rs:257-271: [1,2,3] + [4,5,6] = [5,7,9]; [3,1] + [1,2] has
    dims [3,2] (values fixed by the broadcast rule: a[i] + b[j])."""
    assert O.broadcast_binary([1, 2, 3], [4, 5, 6], "add").tolist() == [5, 7, 9]
    c = O.broadcast_binary(np.array([[1], [2], [3]], np.float32), np.array([[10, 20]], np.float32), "add")
    assert c.shape == (3, 2)
    assert c.tolist() == [[11, 21], [12, 22], [13, 23]]


@pytest.mark.parametrize("sa,sb", [((4, 1, 3), (2, 3)), ((5,), ()), ((), (2, 2)), ((3, 1), (1, 4)),
                                   ((2, 3, 4), (3, 1)), ((1, 1, 7), (6, 1, 1)), ((2, 0, 3), (1, 3)),
                                   ((6, 5), (6, 5)), ((1,), (1, 1, 1))])
@pytest.mark.parametrize("op", ["add", "mul"])
def test_broadcast_binary_matches_numpy(sa, sb, op):
    """Each element is one IEEE float32 add or multiply of the broadcast
    operands, so numpy broadcasting gives the same bits; a dropped or
    swapped stride would fetch the wrong element."""
    rng = np.random.default_rng(len(sa) * 10 + len(sb))
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    want = (np.add if op == "add" else np.multiply)(a, b)
    got = O.broadcast_binary(a, b, op)
    assert got.shape == want.shape
    np.testing.assert_array_equal(got, want)


def test_broadcast_binary_rejects_incompatible():
    with pytest.raises(ValueError):
        O.broadcast_binary(np.zeros((2, 3), np.float32), np.zeros((4,), np.float32), "add")


def test_transpose_last2_index_map():
    x = np.arange(2 * 3 * 5, dtype=np.float32).reshape(2, 3, 5)
    t = O.transpose_last2(x)
    assert t.shape == (2, 5, 3)
    for bi in range(2):
        for i in range(3):
            for j in range(5):
                assert t[bi, j, i] == x[bi, i, j]


def test_linear_integer_inputs_exact():
    """Linear::forward (ghostflow-nn/src/linear.rs:56-69): x W^T + b."""
    rng = np.random.default_rng(3)
    x = rng.integers(-5, 6, size=(16, 64))
    w = rng.integers(-5, 6, size=(48, 64))
    b = rng.integers(-5, 6, size=(48,))
    got = O.linear_forward(x.astype(np.float32), w.astype(np.float32), b.astype(np.float32))
    np.testing.assert_array_equal(got, (x @ w.T + b).astype(np.float32))
    got = O.linear_forward(x.astype(np.float32), w.astype(np.float32), None)
    np.testing.assert_array_equal(got, (x @ w.T).astype(np.float32))


def test_linear_bias_added_after_sum():
    """The bias is a separate broadcast add after the full k-sum
    (arithmetic.rs:124-215): 2^24 + 1 (sum) then + 1 (bias) -> 2^24 + 0 + 0
    ... i.e. the sum 2^24 + 1 rounds to 2^24, then + 1 rounds to 2^24 again."""
    x = np.array([[2.0 ** 24, 1.0]], np.float32)
    w = np.array([[1.0, 1.0]], np.float32)
    b = np.array([1.0], np.float32)
    assert O.linear_forward(x, w, b).item() == 2.0 ** 24


# ---------------------------------------------------------------------------
# softmax (ghostflow-core/src/ops/activation.rs:165-216)
# ---------------------------------------------------------------------------

def test_softmax_reference_known_answers():
    # activation.rs:266-272 (sum within 1e-3) and test_optimizations.rs:51-62
    for data, tol in (([1.0, 2.0, 3.0], 1e-3), ([1.0, 2.0, 3.0, 4.0], 1e-5)):
        y = O.softmax_lastdim(np.array([data], np.float32))
        assert abs(float(y.astype(np.float64).sum()) - 1.0) < tol
        assert (y > 0).all()


def test_softmax_constant_row_uniform():
    y = O.softmax_lastdim(np.full((3, 8), 2.5, np.float32))
    np.testing.assert_array_equal(y, np.full((3, 8), 0.125, np.float32))


@pytest.mark.parametrize("cols", [3, 100, 2048])
def test_softmax_fp64_bound(cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((5, cols)) * 3).astype(np.float32)
    y = O.softmax_lastdim(x).astype(np.float64)
    d = (x - x.max(-1, keepdims=True)).astype(np.float64)  # the f32 subtraction both sides do
    e = np.exp(d)
    exact = e / e.sum(-1, keepdims=True)
    # expf <= 1 ulp, sequential sum (cols roundings), one division
    tol = (4 + cols) * EPS
    assert (np.abs(y - exact) / exact).max() <= tol


def test_softmax_masked_entries_and_dead_rows():
    x = np.array([[0.0, -np.inf, 0.0], [-np.inf, -np.inf, -np.inf]], np.float32)
    y = O.softmax_lastdim(x)
    assert y[0].tolist() == [0.5, 0.0, 0.5]
    assert np.isnan(y[1]).all()  # max = -inf, exp(-inf - -inf) = NaN


# ---------------------------------------------------------------------------
# attention (ghostflow-nn/src/attention.rs:11-64, ghostflow-cuda/src/ops.rs:166-224)
# ---------------------------------------------------------------------------

def _ref_attn_fp64(q, k, v, scale, causal):
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    s = q @ np.swapaxes(k, -1, -2) * scale
    if causal:
        S = s.shape[-1]
        s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return p @ v


def test_sdpa_scale_constant():
    """scale = 1.0 / (128 as f32).sqrt() (attention.rs:19-20) has the bits of
    the correctly rounded 1/sqrt(128)."""
    s = np.float32(1.0) / np.sqrt(np.float32(128.0))
    assert s.view(np.uint32) == 0x3DB504F3


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_fp64(causal):
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((2, 19, 16)).astype(np.float32) for _ in range(3))
    sc = np.float32(1.0) / np.sqrt(np.float32(16))
    got = O.flash_attention(q, k, v, sc, causal)
    ref = _ref_attn_fp64(q, k, v, float(sc), causal)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_flash_attention_causal_closed_forms():
    rng = np.random.default_rng(5)
    s, d = 24, 8
    q = rng.standard_normal((1, s, d)).astype(np.float32)
    v = rng.standard_normal((1, s, d)).astype(np.float32)
    k = rng.standard_normal((1, s, d)).astype(np.float32)
    out = O.flash_attention(q, k, v, 0.25, True)
    np.testing.assert_array_equal(out[0, 0], v[0, 0])  # row 0 sees only key 0
    kc = np.tile(k[:, :1], (1, s, 1))  # constant keys -> prefix mean of V
    out = O.flash_attention(q, kc, v, 0.25, True)
    pm = np.cumsum(v[0].astype(np.float64), 0) / np.arange(1, s + 1)[:, None]
    assert np.abs(out[0] - pm).max() <= 1e-5


def test_sdpa_cycled_causal_mask_equals_causal_flag():
    rng = np.random.default_rng(6)
    bh, s, d = 3, 13, 8
    q, k, v = (rng.standard_normal((bh, s, d)).astype(np.float32) for _ in range(3))
    mask = np.tril(np.ones((s, s), np.float32))
    o1, w1 = O.sdpa(q, k, v, mask=mask, want_weights=True)
    o2 = O.flash_attention(q, k, v, np.float32(1.0) / np.sqrt(np.float32(d)), True)
    np.testing.assert_array_equal(o1, o2)
    assert (w1[:, np.triu_indices(s, 1)[0], np.triu_indices(s, 1)[1]] == 0).all()
    np.testing.assert_allclose(w1.sum(-1), 1.0, rtol=1e-6)


def test_sdpa_mask_is_cycled_over_flat_scores():
    """attention.rs:51-64 cycles the flattened mask over all scores, so a
    29-element mask lands on different (i, j) in each slice."""
    rng = np.random.default_rng(7)
    bh, s, d = 2, 6, 4
    q, k, v = (rng.standard_normal((bh, s, d)).astype(np.float32) for _ in range(3))
    mask = (rng.random(29) > 0.4).astype(np.float32)
    mask[0] = 1.0
    _, w = O.sdpa(q, k, v, mask=mask, want_weights=True)
    flat_keep = mask[np.arange(bh * s * s) % 29] > 0.5
    wf = w.reshape(-1)
    assert (wf[~flat_keep] == 0).all()
    rows_alive = flat_keep.reshape(bh * s, s).any(1)
    assert (wf.reshape(bh * s, s)[rows_alive] > 0).sum() == flat_keep.reshape(bh * s, s)[rows_alive].sum()


def test_flash_attention_rows_matches_full():
    rng = np.random.default_rng(8)
    s, d = 40, 16
    q, k, v = (rng.standard_normal((s, d)).astype(np.float32) for _ in range(3))
    full = O.flash_attention(q[None], k[None], v[None], 0.25, True)[0]
    part = O.flash_attention_rows(q, k, v, 0.25, True, 7, 23)
    np.testing.assert_array_equal(part, full[7:23])


# ---------------------------------------------------------------------------
# quantization (ghostflow-nn/src/quantization.rs:77-204)
# ---------------------------------------------------------------------------

def f32bits(x):
    return int(np.float32(x).view(np.uint32))


def test_per_tensor_symmetric_known_codes():
    """Reference test input [1..6] (quantization.rs:300-324): scale =
    6/127 = 0.047244094; 3/scale = 63.5 exactly and rounds half AWAY from
    zero to 64 (half-even would give 64 too, so 1.0 and 5.0 discriminate:
    21.166 -> 21, 105.83 -> 106)."""
    x = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    q, s, z = O.quantize_per_tensor(x, True)
    assert f32bits(s) == f32bits(np.float32(6.0) / np.float32(127.0))
    assert abs(float(s) - 0.047244094) < 1e-9 and z == 0
    assert q.reshape(-1).tolist() == [21, 42, 64, 85, 106, 127]
    r = O.dequantize(q, np.array([s]), np.array([z]))
    assert np.abs(r - x).max() < 0.1  # the reference's round-trip bound


def test_per_channel_known_codes():
    """quantization.rs:326-350: rows [1,2,3] and [10,20,30], two scales."""
    x = np.array([[1, 2, 3], [10, 20, 30]], np.float32)
    q, s, z = O.quantize_per_channel(x, True)
    assert len(s) == 2
    assert f32bits(s[0]) == f32bits(np.float32(3) / np.float32(127))
    assert f32bits(s[1]) == f32bits(np.float32(30) / np.float32(127))
    assert abs(float(s[0]) - 0.023622047) < 1e-9 and abs(float(s[1]) - 0.23622048) < 1e-8
    assert q.tolist() == [[42, 85, 127], [42, 85, 127]]
    assert (z == 0).all()
    assert np.abs(O.dequantize(q, s, z) - x).max() < 0.5


def test_asymmetric_zero_point():
    """quantization.rs:352-371, [-5,-3,-1,1,3,5] asymmetric: scale =
    fl(10/255) = 0.039215688 (slightly above 10/255), so fl(5/scale) =
    127.49999 and fl(127.49999 - 128) = -0.50000763, which rounds to
    zp = -1 (truncation would give 0)."""
    x = np.array([-5, -3, -1, 1, 3, 5], np.float32)
    q, s, z = O.quantize_per_tensor(x, False)
    assert f32bits(s) == f32bits(np.float32(10) / np.float32(255))
    t = np.float32(np.float32(5.0) / s)
    assert f32bits(t) == f32bits(127.49999237060547)
    assert int(z) == -1
    assert q.tolist() == [-128, -78, -27, 25, 76, 126]
    assert np.abs(O.dequantize(q, np.array([s]), np.array([z])) - x).max() < 0.1


def test_round_half_away_from_zero():
    """f32::round is half away from zero: with absmax 127 the symmetric
    scale is exactly 1.0, so x = +-2.5 and +-0.5 are exact ties; half-even
    would give +-2 and 0."""
    x = np.array([2.5, -2.5, 0.5, -0.5, 127.0, 1.5], np.float32)
    q, s, z = O.quantize_per_tensor(x, True)
    assert float(s) == 1.0 and int(z) == 0
    assert q.tolist() == [3, -3, 1, -1, 127, 2]


def test_asymmetric_zero_point_saturates():
    """DynamicQuantization's activation input [0.5,1.5,2.5]
    (quantization.rs:413-427): -min/scale - 128 = -191.25 saturates the
    `as i8` cast to -128."""
    q, s, z = O.quantize_per_tensor(np.array([0.5, 1.5, 2.5], np.float32), False)
    assert int(z) == -128
    assert f32bits(s) == f32bits(np.float32(2.0) / np.float32(255))
    assert q.tolist() == [-64, 63, 127]


def test_all_zero_input_gives_zero_codes():
    """scale = 0 -> x/scale = NaN -> `as i32` = 0 -> q = 0 (and zp)."""
    for sym in (True, False):
        q, s, z = O.quantize_per_tensor(np.zeros(8, np.float32), sym)
        assert float(s) == 0.0 and (q == 0).all()


def test_per_channel_1d_gives_one_scale_per_element():
    """QAT default config (per-channel, quantization.rs:28-36) on a 1-D
    tensor: shape[0] = numel channels of one element, each quantized to 127
    (test_quantization_aware_training, :386-404)."""
    x = np.array([1, 2, 3, 4], np.float32)
    q, s, z = O.quantize_per_channel(x, True)
    assert q.tolist() == [127] * 4
    assert np.abs(O.dequantize(q, s, z) - x).max() < 0.1


def test_quantize_codes_bracket_and_round_trip():
    """Random data, both schemes: dequantized codes lie within scale/2 of x
    (except clamped ends), and the code is the nearest admissible integer."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((37, 129)) * 0.02).astype(np.float32)
    for sym in (True, False):
        q, s, z = O.quantize_per_channel(x, sym)
        for r in range(37):
            ideal = x[r].astype(np.float64) / np.float64(s[r]) + int(z[r])
            diff = np.abs(q[r].astype(np.float64) - ideal)
            clamped = (q[r] == -128) | (q[r] == 127)
            assert (diff[~clamped] <= 0.5 + 1e-4).all()
        deq = O.dequantize(q, s, z).astype(np.float64)
        err = np.abs(deq - x)
        clamped = (q == -128) | (q == 127)
        assert ((err <= s.astype(np.float64)[:, None] * 0.5001 + 1e-12) | clamped).all()


def test_dequantize_is_one_rounding():
    """(q - zp) is an exact small integer in f32, so (q - zp) * scale is the
    correctly rounded f64 product."""
    rng = np.random.default_rng(10)
    q = rng.integers(-128, 128, size=(5, 33)).astype(np.int8)
    s = rng.random(5).astype(np.float32)
    z = rng.integers(-128, 128, size=5).astype(np.int8)
    got = O.dequantize(q, s, z)
    want = ((q.astype(np.float64) - z[:, None]) * s.astype(np.float64)[:, None]).astype(np.float32)
    np.testing.assert_array_equal(got, want)
    got1 = O.dequantize(q, s[:1], z[:1])
    want1 = ((q.astype(np.float64) - z[0]) * np.float64(s[0])).astype(np.float32)
    np.testing.assert_array_equal(got1, want1)


# ---------------------------------------------------------------------------
# INT8 linear (defined on the reference scheme)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("per_row", [False, True])
def test_qlinear_acc_brute_force_and_epilogue(per_row):
    rng = np.random.default_rng(11)
    m, n, k = 5, 48, 64
    qx = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    g = m if per_row else 1
    sx = (rng.random(g) * 0.1).astype(np.float32)
    zx = rng.integers(-128, 128, size=g).astype(np.int8)
    sw = (rng.random(n) * 0.01).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    y, acc = O.qlinear_i8(qx, sx if per_row else sx[0], zx if per_row else zx[0], per_row, qw, sw, b)
    zcol = (zx if per_row else np.repeat(zx, m)).astype(np.int64)[:, None]
    brute = (qx.astype(np.int64) - zcol) @ qw.astype(np.int64).T
    np.testing.assert_array_equal(acc, brute.astype(np.int32))
    scol = (sx if per_row else np.repeat(sx, m)).astype(np.float64)[:, None]
    exact = brute * scol * sw.astype(np.float64)[None, :] + b.astype(np.float64)
    # three f32 roundings (sx*sw, acc*s, +b) and the f32 rounding of acc
    tol = 4 * EPS * (np.abs(brute * scol * sw.astype(np.float64)) + np.abs(b)) + 1e-30
    assert (np.abs(y - exact) <= tol).all()


def test_qlinear_matches_reference_composite():
    """The reference's executable INT8 path: dequantize both operands and run
    the fp32 matmul (DynamicQuantization::get_weights, quantization.rs:
    275-277).  The integer GEMM equals it within the GEMM error bound."""
    rng = np.random.default_rng(12)
    m, n, k = 7, 40, 96
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    qx, sx, zx = O.quantize_per_tensor(x, False)
    qw, sw, zw = O.quantize_per_channel(w, True)
    assert (zw == 0).all()
    y, _ = O.qlinear_i8(qx, sx, zx, False, qw, sw)
    comp = O.matmul(O.dequantize(qx, np.array([sx]), np.array([zx])), O.dequantize(qw, sw, zw).T.copy())
    bound = 1e-4 * np.sqrt(k) * np.abs(x).max() * np.abs(w).max() * 4
    assert np.abs(y - comp).max() <= bound


# ---------------------------------------------------------------------------
# matmul_backward (ghostflow-autograd/src/backward.rs:131-160)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (33, 17, 29), (64, 48, 80)])
def test_matmul_backward_integer_exact(m, k, n):
    rng = np.random.default_rng(m * 101 + k * 7 + n)
    g = rng.integers(-8, 9, size=(m, n))
    a = rng.integers(-8, 9, size=(m, k))
    b = rng.integers(-8, 9, size=(k, n))
    ga, gb = O.matmul_backward(g.astype(np.float32), a.astype(np.float32), b.astype(np.float32))
    np.testing.assert_array_equal(ga, (g @ b.T).astype(np.float32))
    np.testing.assert_array_equal(gb, (a.T @ g).astype(np.float32))


def test_matmul_backward_sums_sequentially():
    """grad_a sums over l = 0..n-1 and grad_b over l = 0..m-1, ascending,
    each add rounded: 2^24 + 1 + 1 -> 2^24, while 1 + 1 + 2^24 -> 2^24 + 2.
    A transposed operand or a swapped loop order changes the result."""
    g = np.array([[2.0 ** 24, 1.0, 1.0]], np.float32)        # [1, 3]
    b = np.ones((1, 3), np.float32)                            # [k=1, n=3]
    a = np.ones((1, 1), np.float32)
    ga, _ = O.matmul_backward(g, a, b)
    assert ga.item() == 2.0 ** 24
    g2 = np.array([[1.0, 1.0, 2.0 ** 24]], np.float32)
    assert O.matmul_backward(g2, a, b)[0].item() == 2.0 ** 24 + 2
    # grad_b: the sum runs over the rows of a and grad
    a = np.array([[2.0 ** 24], [1.0], [1.0]], np.float32)     # [m=3, k=1]
    g = np.ones((3, 1), np.float32)
    b = np.ones((1, 1), np.float32)
    assert O.matmul_backward(g, a, b)[1].item() == 2.0 ** 24
    a = np.array([[1.0], [1.0], [2.0 ** 24]], np.float32)
    assert O.matmul_backward(g, a, b)[1].item() == 2.0 ** 24 + 2


def test_matmul_backward_fp64_and_adjoint():
    """fp64 brute force within the fp32 GEMM rounding bound, and the adjoint
    identity <grad, A.dB + dA.B> = <grad_a, dA> + <grad_b, dB> that defines
    the gradient of C = A.B."""
    rng = np.random.default_rng(5)
    m, k, n = 40, 30, 50
    g, a, b = (rng.standard_normal(s).astype(np.float32) for s in ((m, n), (m, k), (k, n)))
    ga, gb = O.matmul_backward(g, a, b)
    g64, a64, b64 = g.astype(np.float64), a.astype(np.float64), b.astype(np.float64)
    assert np.abs(ga - g64 @ b64.T).max() <= n * EPS * (np.abs(g64) @ np.abs(b64).T).max()
    assert np.abs(gb - a64.T @ g64).max() <= m * EPS * (np.abs(a64).T @ np.abs(g64)).max()
    da, db = rng.standard_normal((m, k)), rng.standard_normal((k, n))
    lhs = np.sum(g64 * (a64 @ db + da @ b64))
    rhs = np.sum(ga * da) + np.sum(gb * db)
    assert abs(lhs - rhs) <= 1e-4 * (abs(lhs) + 1)


def test_matmul_backward_shape_check():
    with pytest.raises(ValueError):
        O.matmul_backward(np.zeros((2, 3), np.float32), np.zeros((2, 4), np.float32), np.zeros((5, 3), np.float32))
