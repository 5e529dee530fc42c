"""Pins the oracle's MultiHeadAttention::forward_with_cache
(ghostflow-nn/src/attention.rs:100-144) on the CPU:
  * an independent fp64 formulation that slices heads by column
    (h*D .. (h+1)*D of the [B, S, E] projections), so a wrong head split or
    merge fails;
  * one head with identity projections reduces to sdpa bit for bit;
  * incremental decoding with a cache (past_key / past_value, mask None)
    reproduces every row of the full causal forward bit for bit -- the
    property the reference's cache exists for -- which pins the
    concatenation order along dim 1 and the returned new keys/values.
"""
import numpy as np
import pytest

from oracle import oracle as O


def _params(rng, e, bias=True):
    ws = [(rng.standard_normal((e, e)) / np.sqrt(e)).astype(np.float32) for _ in range(4)]
    bs = [(rng.standard_normal(e) * 0.1).astype(np.float32) if bias else None for _ in range(4)]
    return ws, bs


def _mha_fp64(query, key, value, ws, bs, h, mask=None, past_key=None, past_value=None):
    f = lambda t: None if t is None else t.astype(np.float64)  # noqa: E731
    (wq, wk, wv, wo), (bq, bk, bv, bo) = [f(w) for w in ws], [f(b) for b in bs]
    lin = lambda x, w, b: x @ w.T + (0.0 if b is None else b)  # noqa: E731
    q, k, v = lin(f(query), wq, bq), lin(f(key), wk, bk), lin(f(value), wv, bv)
    if past_key is not None:
        k = np.concatenate([f(past_key), k], axis=1)
        v = np.concatenate([f(past_value), v], axis=1)
    b, s, e = q.shape
    skv, d = k.shape[1], e // h
    out = np.zeros((b, s, e))
    wts = np.zeros((b, h, s, skv))
    for bi in range(b):
        for hh in range(h):
            cols = slice(hh * d, (hh + 1) * d)
            sc = q[bi, :, cols] @ k[bi, :, cols].T / np.sqrt(d)
            if mask is not None:
                flat = ((bi * h + hh) * s + np.arange(s)[:, None]) * skv + np.arange(skv)[None, :]
                sc = np.where(mask.reshape(-1)[flat % mask.size] > 0.5, sc, -np.inf)
            p = np.exp(sc - sc.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            wts[bi, hh] = p
            out[bi, :, cols] = p @ v[bi, :, cols]
    return lin(out, wo, bo), wts


@pytest.mark.parametrize("with_past,with_mask", [(False, False), (True, False), (True, True)])
def test_mha_fp64(with_past, with_mask):
    rng = np.random.default_rng(11 + 2 * with_past + with_mask)
    b, s, p, e, h = 2, 3, 4, 8, 2
    ws, bs = _params(rng, e)
    query, key, value = (rng.standard_normal((b, s, e)).astype(np.float32) for _ in range(3))
    pk = rng.standard_normal((b, p, e)).astype(np.float32) if with_past else None
    pv = rng.standard_normal((b, p, e)).astype(np.float32) if with_past else None
    skv = s + (p if with_past else 0)
    mask = None
    if with_mask:
        mask = (rng.random(s * skv) > 0.3).astype(np.float32)
        mask[::skv + 1] = 1.0  # no row fully masked
    out, w, kn, vn = O.mha_forward_with_cache(query, key, value, *ws[:1], bs[0], ws[1], bs[1], ws[2], bs[2],
                                              ws[3], bs[3], h, mask=mask, past_key=pk, past_value=pv)
    ref_out, ref_w = _mha_fp64(query, key, value, ws, bs, h, mask, pk, pv)
    assert out.shape == (b, s, e) and w.shape == (b, h, s, skv) and kn.shape == (b, s, e)
    assert np.abs(out - ref_out).max() <= 1e-5 * np.abs(ref_out).max()
    assert np.abs(w - ref_w).max() <= 1e-5
    kref = key.astype(np.float64) @ ws[1].T.astype(np.float64) + bs[1]
    assert np.abs(kn - kref).max() <= 1e-5 * np.abs(kref).max()


def test_mha_single_head_identity_is_sdpa():
    rng = np.random.default_rng(12)
    b, s, p, e = 2, 5, 3, 16
    eye = np.eye(e, dtype=np.float32)
    query, key, value = (rng.standard_normal((b, s, e)).astype(np.float32) for _ in range(3))
    pk, pv = (rng.standard_normal((b, p, e)).astype(np.float32) for _ in range(2))
    out, w, kn, vn = O.mha_forward_with_cache(query, key, value, eye, None, eye, None, eye, None, eye, None, 1,
                                              past_key=pk, past_value=pv)
    np.testing.assert_array_equal(kn, key)
    np.testing.assert_array_equal(vn, value)
    kc, vc = np.concatenate([pk, key], 1), np.concatenate([pv, value], 1)
    ref, ref_w = O.sdpa(query[:, None], kc[:, None], vc[:, None], want_weights=True)
    np.testing.assert_array_equal(out, ref[:, 0])
    np.testing.assert_array_equal(w, ref_w)


def test_mha_cached_decode_reproduces_full_causal_forward():
    rng = np.random.default_rng(13)
    b, s, e, h = 2, 7, 16, 4
    ws, bs = _params(rng, e)
    x = rng.standard_normal((b, s, e)).astype(np.float32)
    args = (ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], ws[3], bs[3], h)
    causal = np.tril(np.ones((s, s), np.float32))
    full, full_w, full_k, full_v = O.mha_forward_with_cache(x, x, x, *args, mask=causal)
    kc = np.zeros((b, 0, e), np.float32)
    vc = np.zeros((b, 0, e), np.float32)
    for t in range(s):
        xt = x[:, t:t + 1]
        out, w, kn, vn = O.mha_forward_with_cache(xt, xt, xt, *args, past_key=kc if t else None,
                                                  past_value=vc if t else None)
        np.testing.assert_array_equal(out[:, 0], full[:, t])
        np.testing.assert_array_equal(w[:, :, 0], full_w[:, :, t, :t + 1])
        assert (full_w[:, :, t, t + 1:] == 0).all()
        np.testing.assert_array_equal(kn[:, 0], full_k[:, t])
        np.testing.assert_array_equal(vn[:, 0], full_v[:, t])
        kc = np.concatenate([kc, kn], 1)
        vc = np.concatenate([vc, vn], 1)
