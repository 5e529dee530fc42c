"""CPU tests that pin the oracle's SwiGLU pieces before they check the GPU.

SwiGLU::forward (ghostflow-nn/src/llama.rs:276-286) is
down_proj(silu(gate_proj(x)) * up_proj(x)) with
silu(x) = x / (1.0 + (-x).exp()) (ghostflow-core/src/ops/activation.rs:117-122)
and an elementwise `mul` (arithmetic.rs:39-45).  The reference holds no test
values for silu or SwiGLU, so the checks below come from the mathematics:
exact special values, an fp64 closed form, and a float32 restatement on
inputs whose expf result is unambiguous, chosen so that the plausible
x * (1 / (1 + e)) form gives different bits.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

F = np.float32


def _silu(x):
    return O.silu_mul(np.asarray(x, F), np.ones(np.shape(x), F))


def test_silu_special_values():
    got = _silu([0.0, -0.0, 20.0, 100.0, -100.0, np.inf, -np.inf, np.nan])
    # 0 / (1 + 1) = +0 (and -0 / 2 = -0)
    assert got[0] == 0 and not np.signbit(got[0])
    assert got[1] == 0 and np.signbit(got[1])
    # exp(-20) ~ 2e-9 < ulp(1)/2, so 1 + e rounds to 1 and silu(x) = x exactly
    assert got[2] == 20.0 and got[3] == 100.0
    # exp(100) overflows to +inf: -100 / inf = -0
    assert got[4] == 0 and np.signbit(got[4])
    assert got[5] == np.inf
    # -inf / (1 + inf) = -inf / inf = NaN, as the reference computes it
    assert np.isnan(got[6]) and np.isnan(got[7])


def test_silu_fp64_closed_form():
    x = np.random.default_rng(0).uniform(-30, 30, 20000).astype(F)
    got = _silu(x).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / (1.0 + np.exp(-xd))
    # negate (exact), expf (<1 ulp), add, divide: a few ulp of the result,
    # plus the add's rounding relative to 1 + e scaled through the quotient
    ulp = np.spacing(np.abs(ref).astype(F)).astype(np.float64)
    assert (np.abs(got - ref) <= 4 * ulp + 1e-45).all()


def _unambiguous_exp(x):
    """float32(exp(-x)) and a mask of the inputs where exp(-x) in fp64 lies
    well inside one float32 rounding interval, so that any expf with < 0.9 ulp
    error returns that value."""
    e64 = np.exp(-x.astype(np.float64))
    e32 = e64.astype(F)
    lo = np.nextafter(e32, F(-np.inf)).astype(np.float64)
    hi = np.nextafter(e32, F(np.inf)).astype(np.float64)
    mid_lo = (lo + e32.astype(np.float64)) / 2
    mid_hi = (hi + e32.astype(np.float64)) / 2
    width = mid_hi - mid_lo
    ok = (e64 - mid_lo > 0.1 * width) & (mid_hi - e64 > 0.1 * width)
    return e32, ok


def test_silu_mul_division_form_bit_exact():
    rng = np.random.default_rng(1)
    x = rng.uniform(-12, 12, 50000).astype(F)
    u = rng.normal(0, 1, x.size).astype(F)
    e32, ok = _unambiguous_exp(x)
    x, u, e32 = x[ok], u[ok], e32[ok]
    with np.errstate(over="ignore"):
        denom = (F(1) + e32).astype(F)
        want = ((x / denom).astype(F) * u).astype(F)
        other = ((x * (F(1) / denom).astype(F)).astype(F) * u).astype(F)
    got = O.silu_mul(x, u)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # the test separates the reference's division from the reciprocal form
    assert (other.view(np.uint32) != want.view(np.uint32)).sum() > 100


def test_mul_is_one_rounding():
    # silu(20) == 20 exactly, so out == fl(20 * u)
    u = np.random.default_rng(2).normal(0, 1, 1000).astype(F)
    got = O.silu_mul(np.full(u.shape, 20.0, F), u)
    np.testing.assert_array_equal(got, (F(20) * u).astype(F))


def test_silu_mul_shape_check():
    with pytest.raises(ValueError):
        O.silu_mul(np.zeros(3, F), np.zeros(4, F))


def _swiglu_f64(x, wg, bg, wu, bu, wd, bd):
    d = lambda a: np.asarray(a, np.float64)  # noqa: E731
    g = d(x) @ d(wg).T + d(bg)
    u = d(x) @ d(wu).T + d(bu)
    h = g / (1.0 + np.exp(-g)) * u
    return h @ d(wd).T + d(bd), h


@pytest.mark.parametrize("m,hid,inter", [(1, 16, 24), (5, 64, 96), (33, 48, 80)])
def test_swiglu_forward_fp64(m, hid, inter):
    rng = np.random.default_rng(m + hid)
    x = rng.normal(0, 1, (m, hid)).astype(F)
    wg, wu = (rng.uniform(-1, 1, (inter, hid)).astype(F) / F(math.sqrt(hid)) for _ in range(2))
    wd = rng.uniform(-1, 1, (hid, inter)).astype(F) / F(math.sqrt(inter))
    bg, bu = (rng.uniform(-0.1, 0.1, inter).astype(F) for _ in range(2))
    bd = rng.uniform(-0.1, 0.1, hid).astype(F)
    y, h = O.swiglu_forward(x, wg, bg, wu, bu, wd, bd)
    y64, h64 = _swiglu_f64(x, wg, bg, wu, bu, wd, bd)
    assert y.shape == (m, hid) and h.shape == (m, inter)
    assert np.abs(h - h64).max() <= 1e-5 * max(1.0, np.abs(h64).max())
    assert np.abs(y - y64).max() <= 1e-5 * max(1.0, np.abs(y64).max())
    # the bias of each projection lands where it belongs: dropping one moves y
    y_nb, _ = O.swiglu_forward(x, wg, bg, wu, bu, wd, np.zeros_like(bd))
    assert np.abs(y_nb - (y64 - bd)).max() <= 1e-5 * max(1.0, np.abs(y64).max())


def test_qswiglu_forward_stages():
    """The int8 SwiGLU: every stage restated with numpy integer arithmetic
    (exact) and the f32 epilogue of the INT8 linear, on the oracle's own
    pinned quantizers."""
    rng = np.random.default_rng(3)
    m, hid, inter = 7, 64, 48
    x = rng.normal(0, 1, (m, hid)).astype(F)
    wg, wu = (rng.normal(0, 0.02, (inter, hid)).astype(F) for _ in range(2))
    wd = rng.normal(0, 0.02, (hid, inter)).astype(F)
    bg, bu = (rng.uniform(-0.01, 0.01, inter).astype(F) for _ in range(2))
    bd = rng.uniform(-0.01, 0.01, hid).astype(F)
    q = {k: O.quantize_per_channel(w, symmetric=True) for k, w in (("g", wg), ("u", wu), ("d", wd))}
    for _, _, z in q.values():
        assert (z == 0).all()
    r = O.qswiglu_forward(x, q["g"][0], q["g"][1], bg, q["u"][0], q["u"][1], bu, q["d"][0], q["d"][1], bd)

    def lin(qa, sa, za, qw, sw, b):
        acc = (qa.astype(np.int64) - int(za)) @ qw.astype(np.int64).T
        s = (F(sa) * sw).astype(F)
        return ((acc.astype(np.int32).astype(F) * s).astype(F) + b).astype(F)

    qx, sx, zx = O.quantize_per_tensor(x, symmetric=False)
    np.testing.assert_array_equal(r["qx"], qx)
    assert r["sx"] == sx and r["zx"] == zx
    np.testing.assert_array_equal(r["gate"], lin(qx, sx, zx, q["g"][0], q["g"][1], bg))
    np.testing.assert_array_equal(r["up"], lin(qx, sx, zx, q["u"][0], q["u"][1], bu))
    np.testing.assert_array_equal(r["h"], O.silu_mul(r["gate"], r["up"]))
    qh, sh, zh = O.quantize_per_tensor(r["h"], symmetric=False)
    np.testing.assert_array_equal(r["qh"], qh)
    np.testing.assert_array_equal(r["y"], lin(qh, sh, zh, q["d"][0], q["d"][1], bd))
    # and the whole layer stays near the fp32 layer on the dequantized weights
    y32, _ = O.swiglu_forward(x, *(O.dequantize(q[k][0], q[k][1], q[k][2]) if i == 0 else b
                                   for k, b in (("g", bg), ("u", bu), ("d", bd)) for i in (0, 1)))
    assert np.abs(r["y"] - y32).max() <= 0.05 * np.abs(y32).max()
