"""GPU parity of the SwiGLU feed-forward block (ghostflow-nn/src/llama.rs:
259-287) against the oracle, stage by stage.

* silu * up: within 4 ulp of the oracle.  The GPU's expf and glibc's may
  differ in the last bit; every other step is one IEEE rounding on both
  sides.  Values that do not depend on expf's last bit (0, +-20, -100,
  +-inf, NaN) are checked exactly.
* fp32 block: h within the fp32 GEMM bound of gate and up carried through
  silu * up; y against the oracle's Linear on the GPU's own h, within the
  GEMM bound (K = inter).
* int8 block: h within 4 ulp of the oracle's silu * up of the oracle's
  (bit-exact) gate and up; y bit-exact against the oracle's quantize +
  INT8 linear of the GPU's own h, and -- where h matches bit for bit --
  bit-exact against the oracle's whole int8 block.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from _util import gemm_tol, rows_parallel, to_dev, to_np

pytestmark = pytest.mark.gpu
F = np.float32


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _ulp_close(got, ref, ulps=4):
    got = np.asarray(got, F)
    ref = np.asarray(ref, F)
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    with np.errstate(invalid="ignore"):
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = ulps * np.spacing(np.abs(ref)).astype(np.float64)
    bad = ~same & ~(err <= bound)
    assert not bad.any(), (int(bad.sum()), got[bad][:5], ref[bad][:5])


def test_silu_mul_special_values(torch_dev):
    g = np.array([0.0, -0.0, 20.0, -20.0, 100.0, -100.0, np.inf, -np.inf, np.nan, 1.0], F)
    u = np.array([1.0, 1.0, 3.0, 1.0, -2.0, 5.0, 1.0, 1.0, 1.0, 0.0], F)
    got = to_np(_gh().silu_mul(to_dev(g, torch_dev), to_dev(u, torch_dev)))
    ref = O.silu_mul(g, u)
    for i in range(9):
        if i == 3:
            continue  # silu(-20) = -20 * e^-20 / (1 + e^-20) depends on expf's last bit
        if np.isnan(ref[i]):
            assert np.isnan(got[i]), i
        else:
            assert got[i] == ref[i] and np.signbit(got[i]) == np.signbit(ref[i]), (i, got[i], ref[i])
    _ulp_close(got, ref)


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (4096, 0), (4099, 1), (11008 * 16 + 3, 3)])
def test_silu_mul_random(torch_dev, n, offset):
    rng = np.random.default_rng(n)
    g = (rng.normal(0, 4, n + offset)).astype(F)
    u = rng.normal(0, 1, n + offset).astype(F)
    gd, ud = to_dev(g, torch_dev), to_dev(u, torch_dev)
    out = _gh().silu_mul(gd[offset:], ud[offset:])  # offset views exercise the scalar path
    _ulp_close(to_np(out), O.silu_mul(g[offset:], u[offset:]))
    # in place over gate
    _gh().silu_mul(gd, ud, out=gd)
    _ulp_close(to_np(gd), O.silu_mul(g, u))


def _fp32_layer(rng, hidden, inter):
    def lin(n_in, n_out):
        w = rng.uniform(-1, 1, (n_out, n_in)).astype(F) * F(math.sqrt(6.0 / n_in))
        b = rng.uniform(-1, 1, n_out).astype(F) * F(1.0 / math.sqrt(n_in))
        return w, b
    return (*lin(hidden, inter), *lin(hidden, inter), *lin(inter, hidden))


@pytest.mark.parametrize("m,hidden,inter", [(1, 64, 96), (5, 128, 352), (8, 256, 512), (64, 256, 520),
                                            (300, 512, 1024), (16, 4096, 11008)])
@pytest.mark.parametrize("bias", [True, False])
def test_swiglu_f32_stages(torch_dev, m, hidden, inter, bias):
    if not bias and hidden > 512:
        pytest.skip("one large shape per bias mode is enough")
    rng = np.random.default_rng(m * 31 + hidden + inter)
    x = rng.normal(0, 1, (m, hidden)).astype(F)
    wg, bg, wu, bu, wd, bd = _fp32_layer(rng, hidden, inter)
    if not bias:
        bg = bu = bd = None
    dev = lambda a: None if a is None else to_dev(a, torch_dev)  # noqa: E731
    y, h = _gh().swiglu(dev(x), dev(wg), dev(bg), dev(wu), dev(bu), dev(wd), dev(bd), want_h=True)
    y, h = to_np(y), to_np(h)

    gate = O.linear_forward(x, wg, bg)
    up = O.linear_forward(x, wu, bu)
    h_ref = O.silu_mul(gate, up)
    tg, tu = gemm_tol(hidden, x, wg), gemm_tol(hidden, x, wu)
    # |d silu / dv| <= 1.1, so |dh| <= 1.1 |up| tg + (|silu(gate)| + 1.1 tg) tu, plus the final roundings
    sg = np.abs(h_ref / np.where(up == 0, 1, up))
    bound = 1.1 * np.abs(up) * tg + (sg + 1.1 * tg) * tu + 4 * np.spacing(np.abs(h_ref))
    assert (np.abs(h.astype(np.float64) - h_ref) <= bound).all(), float(np.abs(h - h_ref).max())

    y_ref = O.linear_forward(h, wd, bd)
    assert np.abs(y - y_ref).max() <= gemm_tol(inter, h, wd), float(np.abs(y - y_ref).max())


def _int8_layer(rng, hidden, inter, bias):
    w = {"g": rng.normal(0, 0.02, (inter, hidden)).astype(F), "u": rng.normal(0, 0.02, (inter, hidden)).astype(F),
         "d": rng.normal(0, 0.02, (hidden, inter)).astype(F)}
    b = {"g": rng.uniform(-0.01, 0.01, inter).astype(F), "u": rng.uniform(-0.01, 0.01, inter).astype(F),
         "d": rng.uniform(-0.01, 0.01, hidden).astype(F)} if bias else {"g": None, "u": None, "d": None}
    q = {}
    for k in "gud":
        codes, scales, _ = O.quantize_per_channel(w[k], symmetric=True)
        q[k] = (codes, scales, b[k])
    return q


# m <= 64: the skinny gate/up kernel (5 x 4096 x 256 splits K over workgroups);
# 65..128: 128 x (64 + 64) tiles; 129..256: 256 x (64 + 64) (hidden % 128 ==
# 64 -> 64-byte stages: m = 200); above 256: 256 x (128 + 128) tiles; hidden
# = 80 (not a multiple of 64) takes the unfused path.
@pytest.mark.parametrize("m,hidden,inter", [(1, 64, 96), (3, 1040, 208), (4, 4096, 11008), (7, 128, 352),
                                            (5, 4096, 256), (16, 4096, 11008), (40, 4096, 1024), (56, 2048, 768),
                                            (7, 256, 9008), (24, 512, 8240),
                                            (64, 256, 512), (70, 80, 208), (100, 256, 208), (200, 192, 320),
                                            (300, 256, 512), (600, 320, 256), (1024, 512, 768)])
@pytest.mark.parametrize("bias", [True, False])
def test_swiglu_i8_stages(torch_dev, m, hidden, inter, bias):
    if not bias and hidden > 512:
        pytest.skip("one large shape per bias mode is enough")
    gh = _gh()
    rng = np.random.default_rng(m * 17 + hidden * 3 + inter)
    x = rng.normal(0, 1, (m, hidden)).astype(F)
    q = _int8_layer(rng, hidden, inter, bias)
    dev = {}
    for k, (codes, scales, b) in q.items():
        cd = to_dev(codes, torch_dev)
        dev[k] = (cd, to_dev(scales, torch_dev), gh.qweight_rowsum(cd), None if b is None else to_dev(b, torch_dev))
    y, h = gh.qswiglu(to_dev(x, torch_dev), dev["g"], dev["u"], dev["d"], want_h=True)
    y, h = to_np(y), to_np(h)

    r = O.qswiglu_forward(x, q["g"][0], q["g"][1], q["g"][2], q["u"][0], q["u"][1], q["u"][2],
                          q["d"][0], q["d"][1], q["d"][2])
    _ulp_close(h, r["h"])
    # the rest of the block on the GPU's own h: bit-exact
    qh, sh, zh = O.quantize_per_tensor(h, symmetric=False)
    y_ref, _ = O.qlinear_i8(qh, sh, zh, False, q["d"][0], q["d"][1], q["d"][2], want_acc=False)
    np.testing.assert_array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    if np.array_equal(h.view(np.uint32), r["h"].view(np.uint32)):
        np.testing.assert_array_equal(y.view(np.uint32), r["y"].view(np.uint32))


@pytest.mark.parametrize("m", [1, 16, 300])
def test_swiglu_f32_mistral_ffn(torch_dev, m):
    """The Mistral-7B feed-forward shape, hidden 4096, intermediate 14336
    (Mistral::new(..., 14336), ghostflow-ml/src/deep/architectures/
    transformer.rs:2021), fp32 with biases: the decode-size (1, 16) and tile
    (300) routes, checked stage by stage as above."""
    rng = np.random.default_rng(m + 14336)
    hidden, inter = 4096, 14336
    x = rng.normal(0, 1, (m, hidden)).astype(F)
    wg, bg, wu, bu, wd, bd = _fp32_layer(rng, hidden, inter)
    dev = lambda a: to_dev(a, torch_dev)  # noqa: E731
    y, h = _gh().swiglu(dev(x), dev(wg), dev(bg), dev(wu), dev(bu), dev(wd), dev(bd), want_h=True)
    y, h = to_np(y), to_np(h)
    gate = rows_parallel(O.linear_forward, x, wg, bg)
    up = rows_parallel(O.linear_forward, x, wu, bu)
    h_ref = O.silu_mul(gate, up)
    tg, tu = gemm_tol(hidden, x, wg), gemm_tol(hidden, x, wu)
    sg = np.abs(h_ref / np.where(up == 0, 1, up))
    bound = 1.1 * np.abs(up) * tg + (sg + 1.1 * tg) * tu + 4 * np.spacing(np.abs(h_ref))
    assert (np.abs(h.astype(np.float64) - h_ref) <= bound).all(), float(np.abs(h - h_ref).max())
    y_ref = rows_parallel(O.linear_forward, h, wd, bd)
    assert np.abs(y - y_ref).max() <= gemm_tol(inter, h, wd), float(np.abs(y - y_ref).max())


@pytest.mark.parametrize("m", [1, 16, 256, 300, 600])
def test_swiglu_i8_mistral_ffn(torch_dev, m):
    """Mistral's 4096 x 14336 feed-forward block in int8 (DynamicQuantization
    codes, biases): skinny gate/up at m <= 64, 256 x (64 + 64) tiles at 256,
    256 x (128 + 128) at 300 and 600.  h within 4 ulp of the oracle's silu * up of its
    bit-exact gate and up; y bit-exact against the oracle's quantize + INT8
    linear of the GPU's own h."""
    gh = _gh()
    hidden, inter = 4096, 14336
    rng = np.random.default_rng(m * 7 + inter)
    x = rng.normal(0, 1, (m, hidden)).astype(F)
    q = _int8_layer(rng, hidden, inter, True)
    dev = {}
    for k, (codes, scales, b) in q.items():
        cd = to_dev(codes, torch_dev)
        dev[k] = (cd, to_dev(scales, torch_dev), gh.qweight_rowsum(cd), to_dev(b, torch_dev))
    y, h = gh.qswiglu(to_dev(x, torch_dev), dev["g"], dev["u"], dev["d"], want_h=True)
    y, h = to_np(y), to_np(h)
    qx, sx, zx = O.quantize_per_tensor(x, symmetric=False)
    zxa = np.atleast_1d(zx)
    lin = lambda r, w: O.qlinear_i8(r, sx, zxa, False, w[0], w[1], w[2], want_acc=False)[0]  # noqa: E731
    gate = rows_parallel(lin, qx, q["g"])
    up = rows_parallel(lin, qx, q["u"])
    _ulp_close(h, O.silu_mul(gate, up))
    qh, sh, zh = O.quantize_per_tensor(h, symmetric=False)
    zha = np.atleast_1d(zh)
    y_ref = rows_parallel(lambda r: O.qlinear_i8(r, sh, zha, False, q["d"][0], q["d"][1], q["d"][2],
                                                 want_acc=False)[0], qh)
    np.testing.assert_array_equal(y.view(np.uint32), y_ref.view(np.uint32))


def test_swiglu_modules(torch_dev):
    """nn.SwiGLU / QuantizedSwiGLU forward = the ops on their parameters,
    with leading dimensions flattened like Linear::forward's [*, in]."""
    import torch
    gh = _gh()
    torch.manual_seed(0)
    layer = gh.SwiGLU(128, 352, device=torch_dev)
    x = torch.randn((2, 3, 128), device=torch_dev)
    y = layer(x)
    assert y.shape == (2, 3, 128)
    want = gh.swiglu(x.reshape(6, 128), *layer.parameters())
    assert torch.equal(y.reshape(6, 128), want)
    ql = layer.quantize()
    yq = ql(x)
    assert yq.shape == (2, 3, 128)
    assert torch.equal(yq.reshape(6, 128), gh.qswiglu(x.reshape(6, 128), ql.gate, ql.up, ql.down))
    # int8 stays near the fp32 layer
    assert float((yq - y).abs().max()) <= 0.05 * float(y.abs().max())


@pytest.mark.parametrize("m", [1, 3])
def test_swiglu_f32_equals_its_linears(torch_dev, m):
    """Gate and up share one grouped row-dot launch up to 4 rows; h and y
    must equal the same Linears and silu * up run as separate calls, bit for
    bit (the row-dot form splits K only inside a workgroup, so grouping
    changes nothing).  From 5 rows the grouped launch is the skinny MFMA
    kernel, whose K split is chosen for the group: test_swiglu_f32_stages
    holds it to the oracle."""
    import torch
    gh = _gh()
    rng = np.random.default_rng(70 + m)
    hidden, inter = 512, 1376
    x = to_dev(rng.normal(0, 1, (m, hidden)).astype(F), torch_dev)
    wg, bg, wu, bu, wd, bd = (to_dev(a, torch_dev) for a in _fp32_layer(rng, hidden, inter))
    y, h = gh.swiglu(x, wg, bg, wu, bu, wd, bd, want_h=True)
    hh = gh.silu_mul(gh.linear(x, wg, bg), gh.linear(x, wu, bu))
    assert torch.equal(h, hh)
    assert torch.equal(y, gh.linear(hh, wd, bd))
