"""Attention over a key/value cache (gfh_kv_attention_f32) on the GPU against
the oracle's scaled_dot_product_attention (ghostflow-nn/src/attention.rs:
11-64) on the same heads gathered into [B, H, S, D].  The cache layout is
the reference's [B, S, E] (reshape_for_attention, :146-150), rows past
kv_len are NaN so that any read of them shows.  Bar: attention within 1e-4
relative (max|err| / max|ref| and per element)."""
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


def _heads(t, h):
    """[B, S, E] -> [B, H, S, D] (the reference's reshape + transpose view)."""
    b, s, e = t.shape
    return np.ascontiguousarray(t.reshape(b, s, h, e // h).transpose(0, 2, 1, 3))


def _case(b, h, d, sq, kv_len, cap, seed):
    rng = np.random.default_rng(seed)
    e = h * d
    q = rng.standard_normal((b, sq, e)).astype(np.float32)
    kc = np.full((b, cap, e), np.nan, np.float32)
    vc = np.full((b, cap, e), np.nan, np.float32)
    kc[:, :kv_len] = rng.standard_normal((b, kv_len, e))
    vc[:, :kv_len] = rng.standard_normal((b, kv_len, e))
    return q, kc, vc


def _ref(q, kc, vc, kv_len, h, mask=None):
    O = _O()
    out, w = O.sdpa(_heads(q, h), _heads(kc[:, :kv_len], h), _heads(vc[:, :kv_len], h), mask=mask,
                    want_weights=True)
    b, _, sq, _ = out.shape
    return np.ascontiguousarray(out.transpose(0, 2, 1, 3)).reshape(b, sq, -1), w


def _causal_mask(sq, kv_len):
    """Bottom-right causal as an explicit [sq, kv_len] mask (query i is
    position kv_len - sq + i); cycled per (b, h) by the reference."""
    i = np.arange(sq)[:, None]
    j = np.arange(kv_len)[None, :]
    return (j <= kv_len - sq + i).astype(np.float32)


@pytest.mark.parametrize("b,h,d,sq,kv_len,cap", [
    (2, 4, 32, 1, 77, 100),      # one split, ragged key count
    (1, 2, 128, 1, 3000, 3001),  # many splits
    (3, 5, 100, 2, 513, 600),    # D < 128: lanes past D
    (2, 3, 4, 3, 40, 40),        # tiny head, 3 queries in a block of 4
    (1, 4, 64, 7, 257, 300),     # two query blocks
])
def test_vs_oracle(torch_dev, b, h, d, sq, kv_len, cap):
    gh = _gh()
    q, kc, vc = _case(b, h, d, sq, kv_len, cap, seed=b * 100 + sq * 10 + d)
    ref, ref_w = _ref(q, kc, vc, kv_len, h)
    got, w = gh.kv_attention(to_dev(q, torch_dev), to_dev(kc, torch_dev), to_dev(vc, torch_dev), kv_len, h,
                             want_weights=True)
    assert_rel(to_np(got), ref)
    assert_rel(to_np(w), ref_w)


@pytest.mark.parametrize("sq,kv_len", [(1, 50), (4, 200), (6, 1500)])
def test_causal_flag_equals_explicit_mask(torch_dev, sq, kv_len):
    gh = _gh()
    b, h, d = 2, 3, 64
    q, kc, vc = _case(b, h, d, sq, kv_len, kv_len + 5, seed=sq + kv_len)
    mask = _causal_mask(sq, kv_len)
    ref, ref_w = _ref(q, kc, vc, kv_len, h, mask=mask)
    dq, dk, dv = (to_dev(t, torch_dev) for t in (q, kc, vc))
    got, w = gh.kv_attention(dq, dk, dv, kv_len, h, causal=True, want_weights=True)
    assert_rel(to_np(got), ref)
    assert_rel(to_np(w), ref_w)
    got2, w2 = gh.kv_attention(dq, dk, dv, kv_len, h, mask=to_dev(mask, torch_dev), want_weights=True)
    np.testing.assert_array_equal(to_np(got2), to_np(got))
    np.testing.assert_array_equal(to_np(w2), to_np(w))


def test_odd_mask_cycles_and_dead_rows(torch_dev):
    """A 37-element mask cycles over the flattened [B, H, Sq, Skv] scores
    (attention.rs:51-64); an all-zero mask kills every row -> NaN, as the
    reference's softmax over all -inf."""
    gh = _gh()
    b, h, d, sq, kv_len = 2, 2, 16, 3, 90
    q, kc, vc = _case(b, h, d, sq, kv_len, kv_len, seed=9)
    rng = np.random.default_rng(10)
    mask = (rng.random(37) > 0.5).astype(np.float32)
    mask[::5] = 1.0
    ref, ref_w = _ref(q, kc, vc, kv_len, h, mask=mask)
    dq, dk, dv = (to_dev(t, torch_dev) for t in (q, kc, vc))
    got, w = gh.kv_attention(dq, dk, dv, kv_len, h, mask=to_dev(mask, torch_dev), want_weights=True)
    g = to_np(got)
    np.testing.assert_array_equal(np.isnan(g), np.isnan(ref))  # the same heads die
    live = ~np.isnan(ref)
    assert live.any()
    assert_rel(g[live], ref[live])
    assert_rel(np.nan_to_num(to_np(w), nan=-1.0), np.nan_to_num(ref_w, nan=-1.0))
    dead = to_np(gh.kv_attention(dq, dk, dv, kv_len, h, mask=to_dev(np.zeros(4, np.float32), torch_dev)))
    assert np.isnan(dead).all()


def test_split_counters_deterministic_across_calls(torch_dev):
    """Many key splits: the last split of each (b, h) merges in split order
    and resets its counter, so repeated calls agree bit for bit."""
    gh = _gh()
    b, h, d, kv_len = 1, 2, 128, 5000
    q, kc, vc = _case(b, h, d, 1, kv_len, kv_len, seed=11)
    dq, dk, dv = (to_dev(t, torch_dev) for t in (q, kc, vc))
    first = to_np(gh.kv_attention(dq, dk, dv, kv_len, h))
    ref, _ = _ref(q, kc, vc, kv_len, h)
    assert_rel(first, ref)
    for _ in range(3):
        np.testing.assert_array_equal(to_np(gh.kv_attention(dq, dk, dv, kv_len, h)), first)


def test_decode_step_llama_shape(torch_dev):
    """One decode step at B=4, H=32, D=128 over 2048 cached positions (the
    benchmark's SDPA head shape), every (b, h) checked."""
    gh = _gh()
    b, h, d, kv_len = 4, 32, 128, 2048
    q = gh.normal((b, 1, h * d), seed=5, tensor_id=0)
    kc = gh.normal((b, kv_len, h * d), seed=5, tensor_id=1)
    vc = gh.normal((b, kv_len, h * d), seed=5, tensor_id=2)
    ref, _ = _ref(q, kc, vc, kv_len, h)
    got = to_np(gh.kv_attention(to_dev(q, torch_dev), to_dev(kc, torch_dev), to_dev(vc, torch_dev), kv_len, h))
    assert_rel(got, ref)
