"""Fused SDPA and row softmax on the GPU against the oracle
(scaled_dot_product_attention / flash_attention / softmax restated).
Bar (north star): attention within 1e-4 relative --
max|err| / max|ref| <= 1e-4 and |err| <= 1e-4 * (|ref| + mean|ref|) per element."""
import numpy as np
import pytest

from _util import assert_rel, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _O():
    from oracle import oracle
    return oracle


def _scale(d):
    return np.float32(1.0) / np.sqrt(np.float32(d))


@pytest.mark.parametrize("s,d", [(8, 16), (37, 16), (64, 128), (130, 64), (200, 32), (77, 20)])
@pytest.mark.parametrize("causal", [True, False])
def test_small_vs_oracle(torch_dev, s, d, causal):
    gh, O = _gh(), _O()
    b, h = 1, 2
    q = gh.normal((b, h, s, d), seed=1, tensor_id=0)
    k = gh.normal((b, h, s, d), seed=1, tensor_id=1)
    v = gh.normal((b, h, s, d), seed=1, tensor_id=2)
    ref = O.flash_attention(q, k, v, _scale(d), causal)
    got = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), causal=causal))
    assert_rel(got, ref)


def test_causal_row0_is_v0(torch_dev):
    """Causal query 0 attends only to key 0: output row 0 == V[0] exactly."""
    gh = _gh()
    q = gh.normal((2, 3, 50, 64), seed=2, tensor_id=0)
    k = gh.normal((2, 3, 50, 64), seed=2, tensor_id=1)
    v = gh.normal((2, 3, 50, 64), seed=2, tensor_id=2)
    got = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), causal=True))
    np.testing.assert_array_equal(got[:, :, 0, :], v[:, :, 0, :])


def test_constant_keys_give_prefix_mean(torch_dev):
    """All keys equal -> uniform weights over the allowed keys, so causal
    output row i is the mean of V[0..i] (closed form)."""
    gh = _gh()
    s, d = 96, 32
    q = gh.normal((1, 1, s, d), seed=3, tensor_id=0)
    k = np.tile(gh.normal((1, 1, 1, d), seed=3, tensor_id=1), (1, 1, s, 1))
    v = gh.normal((1, 1, s, d), seed=3, tensor_id=2)
    got = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), causal=True))
    ref = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, s + 1)[None, None, :, None]
    assert_rel(got, ref)


def test_weights_and_mask_match_reference_sdpa(torch_dev):
    """attention.rs:11-49 with a [S,S] 1/0 causal mask cycled over the scores,
    returning (output, weights)."""
    gh, O = _gh(), _O()
    b, h, s, d = 2, 2, 45, 32
    q = gh.normal((b, h, s, d), seed=4, tensor_id=0)
    k = gh.normal((b, h, s, d), seed=4, tensor_id=1)
    v = gh.normal((b, h, s, d), seed=4, tensor_id=2)
    mask = np.tril(np.ones((s, s), np.float32))
    ref_o, ref_w = O.sdpa(q, k, v, mask=mask, want_weights=True)
    o, w = gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), mask=to_dev(mask, torch_dev),
                   want_weights=True)
    assert_rel(to_np(o), ref_o)
    np.testing.assert_allclose(to_np(w), ref_w, rtol=1e-4, atol=1e-6)
    assert (to_np(w)[..., np.triu_indices(s, 1)[0], np.triu_indices(s, 1)[1]] == 0).all()
    # the causal flag gives the same result as the cycled causal mask
    oc, wc = gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), causal=True,
                     want_weights=True)
    np.testing.assert_array_equal(to_np(oc), to_np(o))
    np.testing.assert_array_equal(to_np(wc), to_np(w))


def test_odd_mask_cycles_and_dead_rows(torch_dev):
    """A mask whose length does not divide S*S is cycled over the flattened
    scores; a row with every key masked gives NaN, as the reference softmax."""
    gh, O = _gh(), _O()
    b, h, s, d = 1, 2, 12, 16
    q = gh.normal((b, h, s, d), seed=5, tensor_id=0)
    k = gh.normal((b, h, s, d), seed=5, tensor_id=1)
    v = gh.normal((b, h, s, d), seed=5, tensor_id=2)
    rng = np.random.default_rng(0)
    mask = (rng.random(29) > 0.3).astype(np.float32)
    ref_o, ref_w = O.sdpa(q, k, v, mask=mask, want_weights=True)
    o, w = gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), mask=to_dev(mask, torch_dev),
                   want_weights=True)
    o, w = to_np(o), to_np(w)
    np.testing.assert_array_equal(np.isnan(o), np.isnan(ref_o))
    ok = ~np.isnan(ref_o)
    assert_rel(np.where(ok, o, 0), np.where(ok, ref_o, 0))
    np.testing.assert_allclose(w, ref_w, rtol=1e-4, atol=1e-6, equal_nan=True)
    # fully masked rows
    zero_mask = np.zeros((s * s,), np.float32)
    zero_mask[s * 2:] = 1.0  # rows 0 and 1 of every slice have no key
    o2 = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev),
                       mask=to_dev(zero_mask, torch_dev)))
    ref2 = O.sdpa(q, k, v, mask=zero_mask)
    assert np.isnan(o2[:, :, :2]).all() and np.isnan(ref2[:, :, :2]).all()
    assert_rel(o2[:, :, 2:], ref2[:, :, 2:])


def test_non_square_kv(torch_dev):
    gh, O = _gh(), _O()
    q = gh.normal((1, 3, 20, 64), seed=6, tensor_id=0)
    k = gh.normal((1, 3, 70, 64), seed=6, tensor_id=1)
    v = gh.normal((1, 3, 70, 64), seed=6, tensor_id=2)
    ref = O.sdpa(q, k, v)
    got = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev)))
    assert_rel(got, ref)


def test_config5_s512_all_slices(torch_dev):
    """Config 5, S=512: Q,K,V [4,32,512,128] ~ N(0,1), causal, all 128 (b,h)
    slices against the oracle."""
    gh, O = _gh(), _O()
    shape = (4, 32, 512, 128)
    q = gh.normal(shape, seed=0, tensor_id=0)
    k = gh.normal(shape, seed=0, tensor_id=1)
    v = gh.normal(shape, seed=0, tensor_id=2)
    got = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), causal=True))
    ref = O.flash_attention(q, k, v, _scale(128), True)
    assert_rel(got, ref)


def test_config5_s2048_sampled_slices(torch_dev):
    """Config 5, S=2048: 8 random (b,h) slices (slices are independent),
    each against the oracle's flash_attention on that slice."""
    gh, O = _gh(), _O()
    shape = (4, 32, 2048, 128)
    q = gh.normal(shape, seed=0, tensor_id=0)
    k = gh.normal(shape, seed=0, tensor_id=1)
    v = gh.normal(shape, seed=0, tensor_id=2)
    got = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), causal=True))
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(0)
    picks = [divmod(int(bh), 32) for bh in rng.choice(128, 8, replace=False)]
    with ThreadPoolExecutor(8) as pool:  # the oracle's C call releases the GIL
        refs = list(pool.map(lambda p: O.flash_attention(q[p], k[p], v[p], _scale(128), True), picks))
    for (bi, hi), ref in zip(picks, refs):
        assert_rel(got[bi, hi], ref)


def test_long_sequence_s4096(torch_dev):
    """S=4096, d=128, causal, 2 (b,h) slices: 128 key tiles per heavy query
    set and 64 workgroups per slice in the balanced-set kernel, against the
    oracle; the last query row is the mean-weighted sum over all 4096 keys."""
    gh, O = _gh(), _O()
    shape = (1, 2, 4096, 128)
    q = gh.normal(shape, seed=3, tensor_id=0)
    k = gh.normal(shape, seed=3, tensor_id=1)
    v = gh.normal(shape, seed=3, tensor_id=2)
    got = to_np(gh.sdpa(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev), causal=True))
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(2) as pool:  # the oracle's C call releases the GIL
        refs = list(pool.map(lambda h: O.flash_attention(q[0, h], k[0, h], v[0, h], _scale(128), True), range(2)))
    for h, ref in enumerate(refs):
        assert_rel(got[0, h], ref)


@pytest.mark.parametrize("rows,cols", [(1, 3), (1, 4), (7, 1000), (300, 2048), (3, 70000), (5, 260), (9, 4096),
                                       (40000, 512), (2, 4100), (9000, 5), (3, 8)])
def test_softmax_vs_oracle(torch_dev, rows, cols):
    """Rows of up to 4096 columns with cols % 4 == 0 take the wave-per-row
    kernel (1-16 vectors per lane, ragged last vector group: 260, 1000), the
    others the workgroup-per-row one; 40000 and 9000 rows exceed one
    launch's grid, so both walk rows with a grid stride."""
    gh, O = _gh(), _O()
    x = gh.normal((rows, cols), 0.0, 3.0, seed=7, tensor_id=0)
    got = to_np(gh.softmax_lastdim(to_dev(x, torch_dev)))
    ref = O.softmax_lastdim(x)
    # North-star bar against the reference restatement: 1e-4 relative per
    # element.  The reference sums the row sequentially in f32 (relative
    # error growing like cols * eps), the GPU in a tree, so the two differ in
    # the last digits for long rows.
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-12)
    # Against the exact softmax of the same f32 differences fl(x - max): the
    # GPU error is exp's few ulp + a tree sum (log2(cols) roundings) + one
    # division.
    d = (x - x.max(-1, keepdims=True)).astype(np.float64)  # f32 subtraction, as both do
    e = np.exp(d)
    exact = e / e.sum(-1, keepdims=True)
    eps = 2.0 ** -24
    tol = (6 + 2 * np.log2(cols)) * eps
    rel = np.abs(got - exact) / exact
    assert rel.max() <= tol, (rel.max(), tol)
    assert np.abs(got.astype(np.float64).sum(-1) - 1).max() < 1e-5


def test_softmax_beyond_the_mall(torch_dev):
    """[20000, 2048]: x and y together (328 MB) exceed the MALL, so the
    wave-per-row kernel takes its nontemporal loads and stores.  Same
    arithmetic as the cached form: the first rows equal, bit for bit, the
    same rows softmaxed in a small call, and a row sample meets the 1e-4 bar
    against the oracle."""
    gh, O = _gh(), _O()
    rows, cols = 20000, 2048
    x = gh.normal((rows, cols), 0.0, 3.0, seed=11, tensor_id=0)
    got = to_np(gh.softmax_lastdim(to_dev(x, torch_dev)))
    small = to_np(gh.softmax_lastdim(to_dev(np.ascontiguousarray(x[:64]), torch_dev)))
    np.testing.assert_array_equal(got[:64].view(np.uint32), small.view(np.uint32))
    pick = np.random.default_rng(0).choice(rows, 256, replace=False)
    np.testing.assert_allclose(got[pick], O.softmax_lastdim(np.ascontiguousarray(x[pick])), rtol=1e-4, atol=1e-12)


@pytest.mark.parametrize("cols", [8, 7, 512])
def test_softmax_special_values(torch_dev, cols):
    """-inf entries get probability 0, a row of only -inf gives NaN (0/0 as
    in the reference), a NaN entry is ignored by the max fold but poisons its
    row's sum -- on both kernels (cols % 4 == 0 and not)."""
    gh, O = _gh(), _O()
    x = gh.normal((4, cols), seed=3, tensor_id=0)
    x[0, 1] = -np.inf
    x[1, :] = -np.inf
    x[2, 0] = np.nan
    x[3, -1] = np.inf
    got = to_np(gh.softmax_lastdim(to_dev(x, torch_dev)))
    ref = O.softmax_lastdim(x)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_allclose(got[ok], ref[ok], rtol=1e-4, atol=1e-12)
    assert got[0, 1] == 0.0


def test_softmax_reference_known_answers(torch_dev):
    """activation.rs:266-272 and tests/test_optimizations.rs:51-62: rows sum
    to 1 and are positive; a constant row is uniform."""
    gh = _gh()
    for data in ([1.0, 2.0, 3.0], [1.0, 2.0, 3.0, 4.0]):
        y = to_np(gh.softmax_lastdim(to_dev(np.array([data], np.float32), torch_dev)))
        assert abs(y.sum() - 1.0) < 1e-5 and (y > 0).all()
    y = to_np(gh.softmax_lastdim(to_dev(np.full((2, 8), 5.0, np.float32), torch_dev)))
    np.testing.assert_array_equal(y, np.full((2, 8), 0.125, np.float32))
