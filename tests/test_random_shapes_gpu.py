"""Seeded random shapes for the main entry points, checked against the
oracle at the bars of the hand-picked cases:
  * gfh_sgemm over all four layouts with alpha / beta / bias, and the
    batched form with the reference's modulo batch indexing: within the fp32
    GEMM bound 1e-4 sqrt(K) max|a| max|b| (scaled by |alpha|);
  * the INT8 linear (per-tensor or per-row x, with or without zero points,
    with or without bias): int32 accumulators and fp32 outputs bit for bit;
  * the decode GEMVs with fp32 and int8 weights: within the GEMM bound of
    x . W (x . dequantize(W) for int8);
  * scaled_dot_product_attention with and without causal masking or a
    cycled explicit mask: within 1e-4 relative;
  * the INT8 linear on fp32 activations (gfh_qlinear_dynamic_i8, one launch
    or two): bit for bit against quantize_activation + the INT8 linear;
  * attention over a KV cache (a few new queries, causal or masked, the
    cache partly filled): within 1e-4 relative of the oracle's SDPA on the
    filled rows;
  * softmax (1e-4 relative per element), per-channel and per-tensor
    quantization (bit for bit), matmul_backward (GEMM bound),
    MultiHeadAttention::forward_with_cache (1e-4 relative),
    FlashAttention::forward's blockwise recurrence (its normwise bar) and
    SwiGLU::forward in fp32 and int8 (the bars of its stage tests).
The shapes are drawn once from fixed seeds, so every run checks the same
cases; they land on ragged tiles, odd K, split-K boundaries and tiny sizes
that the hand-picked shapes may not."""
import numpy as np
import pytest

from _util import assert_rel, gemm_tol, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _O():
    from oracle import oracle
    return oracle


def _dim(rng, lo, hi):
    """Mostly uniform in [lo, hi], sometimes a small or a power-of-two-ish
    size, the edges the kernels' tiling cares about."""
    r = rng.random()
    if r < 0.2:
        return int(rng.integers(lo, min(hi, lo + 7) + 1))
    if r < 0.35:
        p = int(rng.choice([16, 32, 64, 128, 256, 512]))
        return int(np.clip(p + rng.integers(-1, 2), lo, hi))
    return int(rng.integers(lo, hi + 1))


def _sgemm_cases():
    rng = np.random.default_rng(20261)
    cases = []
    for _ in range(32):
        cases.append((_dim(rng, 1, 600), _dim(rng, 1, 600), _dim(rng, 1, 520), bool(rng.integers(2)),
                      bool(rng.integers(2)), float(rng.choice([1.0, 0.7, -1.3])), float(rng.choice([0.0, 0.5])),
                      bool(rng.integers(2))))
    return cases


@pytest.mark.parametrize("m,n,k,ta,tb,alpha,beta,bias", _sgemm_cases())
def test_sgemm_random(torch_dev, m, n, k, ta, tb, alpha, beta, bias):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(m * 1000003 + n * 1009 + k)
    a = rng.normal(0, 1, (k, m) if ta else (m, k)).astype(np.float32)
    b = rng.normal(0, 1, (n, k) if tb else (k, n)).astype(np.float32)
    c0 = rng.normal(0, 1, (m, n)).astype(np.float32)
    bv = rng.uniform(-0.5, 0.5, n).astype(np.float32) if bias else None
    out = to_dev(c0, torch_dev)
    gh.sgemm(to_dev(a, torch_dev), to_dev(b, torch_dev), trans_a=ta, trans_b=tb, alpha=alpha, beta=beta,
             bias=None if bv is None else to_dev(bv, torch_dev), out=out)
    opa = np.ascontiguousarray(a.T) if ta else a
    opb = np.ascontiguousarray(b.T) if tb else b
    ref = np.float32(alpha) * O.matmul(opa, opb).astype(np.float64)
    if beta:
        ref = ref + np.float32(beta) * c0.astype(np.float64)
    if bv is not None:
        ref = ref + bv
    tol = abs(alpha) * gemm_tol(k, a, b) + 4 * float(np.spacing(np.float32(np.abs(ref).max(initial=1.0))))
    assert np.abs(to_np(out) - ref).max() <= tol


def _batched_cases():
    rng = np.random.default_rng(20262)
    cases = []
    for _ in range(10):
        batch = int(rng.integers(1, 5))
        ba = int(rng.choice([1, batch]))
        bb = int(rng.choice([1, batch])) if ba == batch else batch
        cases.append((ba, bb, _dim(rng, 1, 200), _dim(rng, 1, 200), _dim(rng, 1, 300)))
    return cases


@pytest.mark.parametrize("ba,bb,m,n,k", _batched_cases())
def test_batched_matmul_random(torch_dev, ba, bb, m, n, k):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(ba * 7 + bb * 131 + m * 17 + n * 3 + k)
    a = rng.normal(0, 1, (ba, m, k)).astype(np.float32)
    b = rng.normal(0, 1, (bb, k, n)).astype(np.float32)
    got = to_np(gh.matmul(to_dev(a, torch_dev), to_dev(b, torch_dev)))
    ref = O.batched_matmul(a, b)
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= gemm_tol(k, a, b)


def _qlinear_cases():
    rng = np.random.default_rng(20263)
    cases = []
    for _ in range(28):
        k = int(rng.choice([_dim(rng, 1, 900), 16 * _dim(rng, 1, 80), 64 * _dim(rng, 1, 40)]))
        cases.append((_dim(rng, 1, 600), _dim(rng, 1, 700), k, bool(rng.integers(2)), bool(rng.integers(2)),
                      bool(rng.integers(2))))
    return cases


@pytest.mark.parametrize("m,n,k,x_per_row,with_zp,with_bias", _qlinear_cases())
def test_qlinear_random(torch_dev, m, n, k, x_per_row, with_zp, with_bias):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(m * 7919 + n * 31 + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    bias = rng.uniform(-0.01, 0.01, n).astype(np.float32) if with_bias else None
    qw, sw, _ = O.quantize_per_channel(w, True)
    qx, sx, zx = O.quantize_per_channel(x, not with_zp) if x_per_row else O.quantize_per_tensor(x, not with_zp)
    zx_arg = np.atleast_1d(zx) if with_zp else None
    ry, racc = O.qlinear_i8(qx, sx, zx_arg, x_per_row, qw, sw, bias)
    d = lambda a: None if a is None else to_dev(np.ascontiguousarray(np.atleast_1d(a)), torch_dev)  # noqa: E731
    y, acc = gh.qlinear(d(qx), d(sx), d(zx_arg), d(qw), d(sw), x_per_row=x_per_row, bias=d(bias), want_acc=True)
    np.testing.assert_array_equal(to_np(acc), racc)
    np.testing.assert_array_equal(to_np(y).view(np.uint32), ry.view(np.uint32))


def _gemv_cases():
    rng = np.random.default_rng(20264)
    return [(int(rng.integers(1, 21)), _dim(rng, 1, 5000), _dim(rng, 1, 3000), bool(rng.integers(2)))
            for _ in range(28)]


@pytest.mark.parametrize("b,k,n,int8", _gemv_cases())
def test_gemv_random(torch_dev, b, k, n, int8):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(b * 100003 + k * 13 + n)
    x = rng.normal(0, 1, (b, k)).astype(np.float32)
    w = rng.normal(0, 0.02, (k, n)).astype(np.float32)
    if int8:
        qw, sc, zp = O.quantize_per_channel(w, bool(rng.integers(2)))
        wd = O.dequantize(qw, sc, zp)
        got = to_np(gh.gemv_w8(to_dev(x, torch_dev), to_dev(qw, torch_dev), to_dev(sc, torch_dev),
                               to_dev(zp, torch_dev)))
    else:
        wd = w
        got = to_np(gh.gemv_f32(to_dev(x, torch_dev), to_dev(w, torch_dev)))
    ref = O.matmul(x, wd)
    assert np.abs(got - ref).max() <= gemm_tol(k, x, wd)


def _sdpa_cases():
    rng = np.random.default_rng(20265)
    cases = []
    for _ in range(28):
        sq = _dim(rng, 1, 300)
        mode = int(rng.integers(3))  # 0 plain, 1 causal (sq == skv), 2 cycled mask
        skv = sq if mode == 1 else _dim(rng, 1, 300)
        cases.append((int(rng.integers(1, 3)), int(rng.integers(1, 4)), sq, skv, 4 * int(rng.integers(1, 33)), mode))
    return cases


@pytest.mark.parametrize("b,h,sq,skv,d,mode", _sdpa_cases())
def test_sdpa_random(torch_dev, b, h, sq, skv, d, mode):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(b * 11 + h * 101 + sq * 1009 + skv * 7 + d)
    q = rng.normal(0, 1, (b, h, sq, d)).astype(np.float32)
    k = rng.normal(0, 1, (b, h, skv, d)).astype(np.float32)
    v = rng.normal(0, 1, (b, h, skv, d)).astype(np.float32)
    mask = None
    if mode == 1:
        mask = np.tril(np.ones((sq, skv), np.float32))  # the causal rule as the reference's explicit mask
    elif mode == 2:
        mask = (rng.random(int(rng.integers(1, 3 * skv + 2))) > 0.3).astype(np.float32)
        mask[0] = 1.0
    dq, dk, dv = (to_dev(a, torch_dev) for a in (q, k, v))
    if mode == 1:
        got = to_np(gh.sdpa(dq, dk, dv, causal=True))
    else:
        got = to_np(gh.sdpa(dq, dk, dv, mask=None if mask is None else to_dev(mask, torch_dev)))
    ref = O.sdpa(q, k, v, mask=mask)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), finite)  # fully masked rows: NaN, as the reference
    if finite.any():
        assert_rel(got[finite], ref[finite])


def _dynamic_cases():
    rng = np.random.default_rng(20266)
    return [(_dim(rng, 1, 40), _dim(rng, 1, 3000), 16 * _dim(rng, 1, 300), bool(rng.integers(2)))
            for _ in range(20)]


@pytest.mark.parametrize("m,n,k,with_bias", _dynamic_cases())
def test_qlinear_dynamic_random(torch_dev, m, n, k, with_bias):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(m * 31 + n * 7 + k)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    bias = rng.uniform(-0.01, 0.01, n).astype(np.float32) if with_bias else None
    qw, sw, _ = O.quantize_per_channel(w, True)
    dqw = to_dev(qw, torch_dev)
    got = to_np(gh.qlinear_dynamic(to_dev(x, torch_dev), dqw, to_dev(sw, torch_dev), gh.qweight_rowsum(dqw),
                                   bias=None if bias is None else to_dev(bias, torch_dev)))
    qx, sx, zx = O.quantize_per_tensor(x, False)
    ref, _ = O.qlinear_i8(qx, sx, zx, False, qw, sw, bias, want_acc=False)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def _kv_cases():
    rng = np.random.default_rng(20267)
    cases = []
    for _ in range(20):
        h = int(rng.integers(1, 19))
        d = 4 * int(rng.integers(1, 33))
        sq = int(rng.integers(1, 17))
        kv_len = int(rng.integers(sq, 700))
        cases.append((int(rng.integers(1, 4)), h, sq, kv_len, kv_len + int(rng.integers(0, 50)), d,
                      int(rng.integers(3))))
    return cases


@pytest.mark.parametrize("b,h,sq,kv_len,cap,d,mode", _kv_cases())
def test_kv_attention_random(torch_dev, b, h, sq, kv_len, cap, d, mode):
    """q [B, Sq, E] over the first kv_len rows of [B, cap, E] caches (head h =
    columns h*D .. h*D+D-1); mode 0 plain, 1 causal (the queries are the last
    Sq positions), 2 a cycled explicit mask."""
    gh, O = _gh(), _O()
    e = h * d
    rng = np.random.default_rng(b * 3 + h * 97 + sq * 1013 + kv_len * 5 + d)
    q = rng.normal(0, 1, (b, sq, e)).astype(np.float32)
    kc = rng.normal(0, 1, (b, cap, e)).astype(np.float32)
    vc = rng.normal(0, 1, (b, cap, e)).astype(np.float32)
    heads = lambda t, s: t[:, :s].reshape(b, s, h, d).transpose(0, 2, 1, 3).copy()  # noqa: E731
    mask = None
    if mode == 1:
        mask = np.ones((sq, kv_len), np.float32)
        for i in range(sq):
            mask[i, kv_len - sq + i + 1:] = 0.0
    elif mode == 2:
        mask = (rng.random(int(rng.integers(1, 2 * kv_len + 2))) > 0.3).astype(np.float32)
        mask[0] = 1.0
    got = gh.ops.kv_attention(to_dev(q, torch_dev), to_dev(kc, torch_dev), to_dev(vc, torch_dev), kv_len, h,
                              causal=mode == 1, mask=to_dev(mask, torch_dev) if mode == 2 else None)
    got = to_np(got).reshape(b, sq, h, d).transpose(0, 2, 1, 3)
    ref = O.sdpa(heads(q, sq), heads(kc, kv_len), heads(vc, kv_len), mask=mask)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), finite)
    if finite.any():
        assert_rel(got[finite], ref[finite])


def _softmax_cases():
    rng = np.random.default_rng(20268)
    return [(_dim(rng, 1, 3000), _dim(rng, 1, 5000)) for _ in range(16)]


@pytest.mark.parametrize("rows,cols", _softmax_cases())
def test_softmax_random(torch_dev, rows, cols):
    """Tensor::softmax(-1): 1e-4 relative per element (the reference sums a
    row sequentially, the GPU in a tree)."""
    gh, O = _gh(), _O()
    x = np.random.default_rng(rows * 7 + cols).normal(0, 3, (rows, cols)).astype(np.float32)
    got = to_np(gh.softmax_lastdim(to_dev(x, torch_dev)))
    np.testing.assert_allclose(got, O.softmax_lastdim(x), rtol=1e-4, atol=1e-12)


def _quant_cases():
    rng = np.random.default_rng(20269)
    return [(_dim(rng, 1, 500), _dim(rng, 1, 3000), bool(rng.integers(2))) for _ in range(16)]


@pytest.mark.parametrize("rows,cols,symmetric", _quant_cases())
def test_quantize_random(torch_dev, rows, cols, symmetric):
    """quantize_per_channel_int8 and quantize_per_tensor_int8: codes, scales
    and zero points bit for bit."""
    gh, O = _gh(), _O()
    x = np.random.default_rng(rows * 13 + cols).normal(0, 2, (rows, cols)).astype(np.float32)
    dx = to_dev(x, torch_dev)
    for got, ref in ((gh.quantize_per_channel(dx, symmetric), O.quantize_per_channel(x, symmetric)),
                     (gh.quantize_per_tensor(dx, symmetric), O.quantize_per_tensor(x, symmetric))):
        q, s, z = (to_np(t) for t in got)
        rq, rs, rz = ref
        np.testing.assert_array_equal(q.reshape(-1), np.asarray(rq).reshape(-1))
        np.testing.assert_array_equal(s.reshape(-1).view(np.uint32),
                                      np.atleast_1d(np.asarray(rs, np.float32)).view(np.uint32))
        np.testing.assert_array_equal(z.reshape(-1), np.atleast_1d(np.asarray(rz, np.int8)))


def _backward_cases():
    rng = np.random.default_rng(20270)
    return [(_dim(rng, 1, 400), _dim(rng, 1, 400), _dim(rng, 1, 400)) for _ in range(12)]


@pytest.mark.parametrize("m,k,n", _backward_cases())
def test_matmul_backward_random(torch_dev, m, k, n):
    """matmul_backward: grad . b^T and a^T . grad within the GEMM bound."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(m * 3 + k * 5 + n * 7)
    g = rng.normal(0, 1, (m, n)).astype(np.float32)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1, (k, n)).astype(np.float32)
    ga, gb = gh.matmul_backward(to_dev(g, torch_dev), to_dev(a, torch_dev), to_dev(b, torch_dev))
    ra, rb = O.matmul_backward(g, a, b)
    assert np.abs(to_np(ga) - ra).max() <= gemm_tol(n, g, b)
    assert np.abs(to_np(gb) - rb).max() <= gemm_tol(m, a, g)


def _mha_cases():
    rng = np.random.default_rng(20271)
    cases = []
    for _ in range(14):
        h = int(rng.integers(1, 9))
        e = h * 4 * int(rng.integers(1, 33))
        sq = int(rng.integers(1, 40))
        cases.append((int(rng.integers(1, 4)), sq, sq, int(rng.integers(0, 60)), e, h, bool(rng.integers(2))))
    return cases


@pytest.mark.parametrize("b,sq,sk,p,e,h,with_mask", _mha_cases())
def test_mha_random(torch_dev, b, sq, sk, p, e, h, with_mask):
    """MultiHeadAttention::forward_with_cache: output and weights within 1e-4
    relative (fully masked rows NaN, as the reference), new keys / values
    within the GEMM bound."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(b * 17 + sq * 101 + p * 7 + e)
    bound, bb = np.sqrt(6.0 / e), 1.0 / np.sqrt(e)
    ws = [rng.uniform(-bound, bound, (e, e)).astype(np.float32) for _ in range(4)]
    bs = [rng.uniform(-bb, bb, e).astype(np.float32) for _ in range(4)]
    params = [t for pair in zip(ws, bs) for t in pair]
    query, key, value = (rng.standard_normal((b, s, e)).astype(np.float32) for s in (sq, sk, sk))
    pk = rng.standard_normal((b, p, e)).astype(np.float32) if p else None
    pv = rng.standard_normal((b, p, e)).astype(np.float32) if p else None
    mask = None
    if with_mask:
        mask = (rng.random(int(rng.integers(1, sq * (p + sk) + 4))) > 0.3).astype(np.float32)
        mask[0] = 1.0
    ref = O.mha_forward_with_cache(query, key, value, *params, h, mask=mask, past_key=pk, past_value=pv)
    dev = lambda t: None if t is None else to_dev(t, torch_dev)  # noqa: E731
    got = gh.mha_forward_with_cache(dev(query), dev(key), dev(value), *[dev(t) for t in params], h,
                                    mask=dev(mask), past_key=dev(pk), past_value=dev(pv))
    out, w = to_np(got[0].contiguous()), to_np(got[1].contiguous())
    live = ~np.isnan(ref[0])
    assert (np.isnan(out) == ~live).all()
    if live.any():
        assert_rel(out[live], ref[0][live])
    assert_rel(np.nan_to_num(w, nan=-1.0), np.nan_to_num(ref[1], nan=-1.0))
    kn = to_np(got[2]).transpose(0, 2, 1, 3).reshape(b, sk, e)
    assert np.abs(kn - ref[2]).max() <= gemm_tol(e, key, ws[1]) + np.abs(bs[1]).max() * 1e-6


def _flash_cases():
    rng = np.random.default_rng(20272)
    cases = []
    for _ in range(12):
        bm = int(rng.choice([1, 7, 16, 32, 64, 100]))
        bn = int(rng.choice([1, 5, 32, 64, 96, 128]))
        sk = _dim(rng, 1, 400)
        if bn == 1:
            sk = min(sk, 300)
        cases.append((int(rng.integers(1, 4)), _dim(rng, 1, 400), sk, int(rng.integers(1, 129)), bm, bn,
                      bool(rng.integers(2)), float(rng.uniform(0.05, 0.5))))
    return cases


@pytest.mark.parametrize("bsz,sq,sk,d,bm,bn,causal,scale", _flash_cases())
def test_flash_attention_blockwise_random(torch_dev, bsz, sq, sk, d, bm, bn, causal, scale):
    """FlashAttention::forward's blockwise recurrence: max|err| <= 1e-4
    max|ref|, and what the reference leaves at exactly 0 is exactly 0."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(bsz * 5 + sq * 11 + sk * 13 + d)
    q, k, v = (rng.normal(0, 1, (bsz, s, d)).astype(np.float32) for s in (sq, sk, sk))
    ref = O.flash_attention_blockwise(q, k, v, bm, bn, causal, scale)
    got = to_np(gh.flash_attention_blockwise(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev),
                                             block_size_m=bm, block_size_n=bn, causal=causal, scale=scale))
    np.testing.assert_array_equal(got == 0.0, ref == 0.0)
    assert float(np.abs(got.astype(np.float64) - ref).max()) <= 1e-4 * float(np.abs(ref).max(initial=0.0))


def _swiglu_cases():
    rng = np.random.default_rng(20273)
    return [(_dim(rng, 1, 700), 16 * _dim(rng, 1, 64), 16 * _dim(rng, 1, 96), bool(rng.integers(2)),
             bool(rng.integers(2))) for _ in range(16)]


@pytest.mark.parametrize("m,hidden,inter,int8,bias", _swiglu_cases())
def test_swiglu_random(torch_dev, m, hidden, inter, int8, bias):
    """SwiGLU::forward.  fp32: h = silu(gate) * up within the bound that the
    GEMM bound of gate and up implies, y within the GEMM bound of h . Wd^T.
    int8 (DynamicQuantization's scheme per Linear): h within 4 ulp of the
    oracle's silu * up of its bit-exact gate and up, y bit for bit against
    the oracle's quantize + INT8 linear of the GPU's own h."""
    gh, O = _gh(), _O()
    rng = np.random.default_rng(m * 19 + hidden * 7 + inter)
    x = rng.normal(0, 1, (m, hidden)).astype(np.float32)
    sc = np.float32(np.sqrt(6.0 / hidden)), np.float32(np.sqrt(6.0 / inter))
    wg = (rng.uniform(-1, 1, (inter, hidden)) * sc[0]).astype(np.float32)
    wu = (rng.uniform(-1, 1, (inter, hidden)) * sc[0]).astype(np.float32)
    wd = (rng.uniform(-1, 1, (hidden, inter)) * sc[1]).astype(np.float32)
    bg, bu, bd = ((rng.uniform(-0.05, 0.05, n).astype(np.float32) if bias else None) for n in (inter, inter, hidden))
    dev = lambda a: None if a is None else to_dev(a, torch_dev)  # noqa: E731
    if not int8:
        y, h = (to_np(t) for t in gh.swiglu(dev(x), dev(wg), dev(bg), dev(wu), dev(bu), dev(wd), dev(bd), want_h=True))
        gate, up = O.linear_forward(x, wg, bg), O.linear_forward(x, wu, bu)
        h_ref = O.silu_mul(gate, up)
        tg, tu = gemm_tol(hidden, x, wg), gemm_tol(hidden, x, wu)
        sg = np.abs(h_ref / np.where(up == 0, 1, up))
        bound = 1.1 * np.abs(up) * tg + (sg + 1.1 * tg) * tu + 4 * np.spacing(np.abs(h_ref))
        assert (np.abs(h.astype(np.float64) - h_ref) <= bound).all()
        assert np.abs(y - O.linear_forward(h, wd, bd)).max() <= gemm_tol(inter, h, wd)
        return
    q = {}
    for name, w, b in (("g", wg, bg), ("u", wu, bu), ("d", wd, bd)):
        codes, scales, _ = O.quantize_per_channel(w, True)
        cd = to_dev(codes, torch_dev)
        q[name] = (codes, scales, b, (cd, to_dev(scales, torch_dev), gh.qweight_rowsum(cd), dev(b)))
    y, h = (to_np(t) for t in gh.qswiglu(dev(x), q["g"][3], q["u"][3], q["d"][3], want_h=True))
    qx, sx, zx = O.quantize_per_tensor(x, symmetric=False)
    lin = lambda w: O.qlinear_i8(qx, sx, np.atleast_1d(zx), False, w[0], w[1], w[2], want_acc=False)[0]  # noqa: E731
    h_ref = O.silu_mul(lin(q["g"]), lin(q["u"]))
    same = (h == h_ref) | (np.isnan(h) & np.isnan(h_ref))
    err = np.abs(h.astype(np.float64) - h_ref.astype(np.float64))
    assert (same | (err <= 4 * np.spacing(np.abs(h_ref)).astype(np.float64))).all()
    qh, sh, zh = O.quantize_per_tensor(h, symmetric=False)
    y_ref, _ = O.qlinear_i8(qh, sh, np.atleast_1d(zh), False, q["d"][0], q["d"][1], q["d"][2], want_acc=False)
    np.testing.assert_array_equal(y.view(np.uint32), y_ref.view(np.uint32))
