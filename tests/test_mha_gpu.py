"""MultiHeadAttention::forward_with_cache (ghostflow-nn/src/attention.rs:
100-144) on the GPU against the oracle's restatement (oracle.
mha_forward_with_cache, pinned in test_mha_oracle.py).  Bars: outputs and
weights within 1e-4 relative (the attention bar); the new keys/values, which
are Linear outputs, within the GEMM bound."""
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


def _params(e, seed):
    rng = np.random.default_rng(seed)
    bound, bb = np.sqrt(6.0 / e), 1.0 / np.sqrt(e)
    ws = [rng.uniform(-bound, bound, (e, e)).astype(np.float32) for _ in range(4)]
    bs = [rng.uniform(-bb, bb, e).astype(np.float32) for _ in range(4)]
    return [a for pair in zip(ws, bs) for a in pair]  # wq, bq, wk, bk, wv, bv, wo, bo


def _dev(arrs, dev):
    return [None if a is None else to_dev(a, dev) for a in arrs]


@pytest.mark.parametrize("b,sq,sk,p,e,h,with_mask", [
    (2, 5, 5, 0, 64, 4, False),    # self-attention, decode kernel (sq <= 16)
    (2, 40, 40, 0, 64, 4, False),  # tiled SDPA on the strided [B, S, E] layout
    (1, 3, 3, 7, 96, 3, True),     # past keys + a cycled mask
    (3, 20, 20, 11, 128, 2, True),  # past, tiled path, D = 64
    (2, 1, 1, 9, 32, 8, False),    # one decode step, D = 4
])
def test_forward_with_cache_vs_oracle(torch_dev, b, sq, sk, p, e, h, with_mask):
    gh, O = _gh(), _O()
    rng = np.random.default_rng(b * 1000 + sq * 10 + p)
    params = _params(e, seed=e + h)
    query = rng.standard_normal((b, sq, e)).astype(np.float32)
    key = rng.standard_normal((b, sk, e)).astype(np.float32)
    value = rng.standard_normal((b, sk, e)).astype(np.float32)
    pk = rng.standard_normal((b, p, e)).astype(np.float32) if p else None
    pv = rng.standard_normal((b, p, e)).astype(np.float32) if p else None
    mask = None
    if with_mask:
        mask = (rng.random(sq * (p + sk) + 3) > 0.3).astype(np.float32)
        mask[::4] = 1.0
    ref = O.mha_forward_with_cache(query, key, value, *params, h, mask=mask, past_key=pk, past_value=pv)
    got = gh.mha_forward_with_cache(*_dev([query, key, value], torch_dev), *_dev(params, torch_dev), h,
                                    mask=None if mask is None else to_dev(mask, torch_dev),
                                    past_key=None if pk is None else to_dev(pk, torch_dev),
                                    past_value=None if pv is None else to_dev(pv, torch_dev))
    out, w, kn, vn = (to_np(t.contiguous()) if i < 2 else to_np(t) for i, t in enumerate(got))
    live = ~np.isnan(ref[0])
    assert (np.isnan(out) == ~live).all()
    assert_rel(out[live], ref[0][live])
    assert_rel(np.nan_to_num(w, nan=-1.0), np.nan_to_num(ref[1], nan=-1.0))
    d = e // h
    # k_cache / v_cache come back as [B, H, Sk, D] views of the new rows
    assert kn.shape == (b, h, sk, d)
    kn = kn.transpose(0, 2, 1, 3).reshape(b, sk, e)
    vn = vn.transpose(0, 2, 1, 3).reshape(b, sk, e)
    assert np.abs(kn - ref[2]).max() <= gemm_tol(e, key, params[2]) + np.abs(params[3]).max() * 1e-6
    assert np.abs(vn - ref[3]).max() <= gemm_tol(e, value, params[4]) + np.abs(params[5]).max() * 1e-6


@pytest.mark.parametrize("sq,p", [(24, 0), (24, 13), (5, 30)])
def test_causal_flag_equals_lower_triangular_mask(torch_dev, sq, p):
    """causal keeps key j for query i when j <= P + Sk - Sq + i: the same
    as passing that mask explicitly, on both attention paths."""
    import torch
    gh, O = _gh(), _O()
    b, e, h = 2, 64, 2
    rng = np.random.default_rng(sq + p)
    params = _params(e, seed=3)
    x = rng.standard_normal((b, sq, e)).astype(np.float32)
    pk = rng.standard_normal((b, p, e)).astype(np.float32)
    pv = rng.standard_normal((b, p, e)).astype(np.float32)
    kv = p + sq
    mask = (np.arange(kv)[None, :] <= p + np.arange(sq)[:, None]).astype(np.float32)
    ref = O.mha_forward_with_cache(x, x, x, *params, h, mask=mask, past_key=pk if p else None,
                                   past_value=pv if p else None)
    dev = _dev(params, torch_dev)
    kc = torch.zeros((b, kv + 4, e), device=torch_dev)
    vc = torch.zeros_like(kc)
    kc[:, :p] = to_dev(pk, torch_dev)
    vc[:, :p] = to_dev(pv, torch_dev)
    dx = to_dev(x, torch_dev)
    dm = to_dev(mask, torch_dev)
    # with the weights output (the 32-query kernel) and without it (the
    # balanced-set kernel): the flag and the mask agree bit for bit on each
    out, w = gh.mha_forward_cached(dx, dx, dx, *dev, h, kc, vc, p, causal=True, want_weights=True)
    assert_rel(to_np(out), ref[0])
    assert_rel(to_np(w), ref[1])
    out_m, w_m = gh.mha_forward_cached(dx, dx, dx, *dev, h, kc, vc, p, mask=dm, want_weights=True)
    np.testing.assert_array_equal(to_np(out_m), to_np(out))
    np.testing.assert_array_equal(to_np(w_m), to_np(w))
    out_c = gh.mha_forward_cached(dx, dx, dx, *dev, h, kc, vc, p, causal=True)
    assert_rel(to_np(out_c), ref[0])
    out2 = gh.mha_forward_cached(dx, dx, dx, *dev, h, kc, vc, p, mask=dm)
    np.testing.assert_array_equal(to_np(out2), to_np(out_c))


def test_incremental_decoding_matches_full_causal_forward(torch_dev):
    """Prefill 6 positions into a KVCache, then decode 5 more one at a time:
    every step's output equals (within the bar) the matching row of one
    causal forward over all 11 positions -- the property the oracle pins bit
    for bit for the reference path."""
    import torch
    gh, O = _gh(), _O()
    b, s, e, h = 2, 11, 128, 4
    rng = np.random.default_rng(17)
    x = rng.standard_normal((b, s, e)).astype(np.float32)
    mha = gh.MultiHeadAttention(e, h, device=torch_dev)
    mha.eval()
    params = _params(e, seed=5)
    for t, a in zip(mha.parameters(), params):
        t.copy_(torch.from_numpy(a))
    full = O.mha_forward_with_cache(x, x, x, *params, h, mask=np.tril(np.ones((s, s), np.float32)))[0]
    cache = gh.KVCache(b, 16, e, device=torch_dev)
    dx = to_dev(x, torch_dev)
    pre = to_np(mha.step(dx[:, :6].contiguous(), cache, causal=True))
    assert_rel(pre, full[:, :6])
    for t in range(6, s):
        y = to_np(mha.step(dx[:, t:t + 1].contiguous(), cache))
        assert_rel(y[:, 0], full[:, t])
    assert cache.length == s


def test_decode_step_llama_shape(torch_dev):
    """One decode step of a 4096-wide, 32-head layer at B=4 over 2047 cached
    positions (LLaMA-7B attention: 32 heads of 128, as in the benchmark's SDPA shape)."""
    import torch
    gh, O = _gh(), _O()
    b, e, h, p = 4, 4096, 32, 2047
    params = [gh.uniform((e, e) if i % 2 == 0 else (e,), -1 / 64, 1 / 64, seed=0, tensor_id=10 + i)
              for i in range(8)]
    x = gh.normal((b, 1, e), seed=0, tensor_id=0)
    pk = gh.normal((b, p, e), seed=0, tensor_id=1)
    pv = gh.normal((b, p, e), seed=0, tensor_id=2)
    ref_out, ref_w, _, _ = O.mha_forward_with_cache(x, x, x, *params, h, past_key=pk, past_value=pv)
    kc = torch.empty((b, p + 1, e), device=torch_dev)
    vc = torch.empty_like(kc)
    kc[:, :p] = to_dev(pk, torch_dev)
    vc[:, :p] = to_dev(pv, torch_dev)
    dx = to_dev(x, torch_dev)
    out, w = gh.mha_forward_cached(dx, dx, dx, *_dev(params, torch_dev), h, kc, vc, p, want_weights=True)
    assert_rel(to_np(out), ref_out)
    assert_rel(to_np(w), ref_w)


def test_module_forward_is_self_attention(torch_dev):
    import torch
    gh, O = _gh(), _O()
    b, s, e, h = 2, 9, 64, 4
    mha = gh.MultiHeadAttention(e, h, dropout=0.1, device=torch_dev)
    x = torch.randn(b, s, e, device=torch_dev)
    with pytest.raises(gh.GhostFlowError):
        mha.forward(x)  # training mode with dropout > 0: not on this path
    mha.eval()
    y = to_np(mha(x))
    params = [to_np(t) for t in mha.parameters()]
    xn = to_np(x)
    assert_rel(y, O.mha_forward_with_cache(xn, xn, xn, *params, h)[0])


@pytest.mark.parametrize("b,sq,sk,p,exact", [
    (4, 1, 1, 300, True),  # a decode step: q, k and v in one grouped row-dot launch
    (1, 3, 3, 5, True),    # one sequence, 3 new rows: grouped as well
    (2, 1, 1, 0, True),    # no past
    (3, 2, 2, 4, True),    # k / v rows strided per batch in the cache: three launches
    (6, 1, 1, 7, False),   # 6 rows: one grouped skinny MFMA launch
    (40, 1, 1, 3, False),  # 40 rows: the same, three row blocks
])
def test_projections_equal_separate_linears(torch_dev, b, sq, sk, p, exact):
    """Where the q / k / v projections share one launch, each must equal the
    same Linear (gfh_sgemm NT) run alone: the cache rows written, and the
    output against Linear -> kv_attention -> Linear composed from separate
    calls.  Bit for bit up to 4 rows (the row-dot form splits K only inside
    a workgroup, so grouping changes nothing) and where the products are not
    grouped; from 5 rows the grouped skinny launch chooses its K split for
    the whole group, so its sums may differ from a lone launch's in the last
    bits: within the GEMM bound, and the output within the attention bar."""
    import torch
    gh = _gh()
    e, h, cap = 256, 4, 16 + 300
    params = _dev(_params(e, 17 + b), torch_dev)
    wq, bq, wk, bk, wv, bv, wo, bo = params
    rng = np.random.default_rng(b * 100 + sq)
    q_in, k_in, v_in = (to_dev(rng.normal(0, 1, (b, s, e)).astype(np.float32), torch_dev) for s in (sq, sk, sk))
    kc = to_dev(rng.normal(0, 1, (b, cap, e)).astype(np.float32), torch_dev)
    vc = to_dev(rng.normal(0, 1, (b, cap, e)).astype(np.float32), torch_dev)
    kc0, vc0 = kc.clone(), vc.clone()
    out = gh.mha_forward_cached(q_in, k_in, v_in, wq, bq, wk, bk, wv, bv, wo, bo, h, kc, vc, p)
    torch.cuda.synchronize()
    if sk == 1 or b == 1:  # the new rows of every batch projected as one [b * sk, e] product
        kn = gh.linear(k_in.reshape(b * sk, e), wk, bk).reshape(b, sk, e)
        vn = gh.linear(v_in.reshape(b * sk, e), wv, bv).reshape(b, sk, e)
    else:  # one [sk, e] product per batch (the rows are strided in the cache)
        kn = torch.stack([gh.linear(k_in[i], wk, bk) for i in range(b)])
        vn = torch.stack([gh.linear(v_in[i], wv, bv) for i in range(b)])
    if exact:
        assert torch.equal(kc[:, p:p + sk], kn) and torch.equal(vc[:, p:p + sk], vn)
    else:
        for got, ref, xin, w in ((kc[:, p:p + sk], kn, k_in, wk), (vc[:, p:p + sk], vn, v_in, wv)):
            tol = gemm_tol(e, to_np(xin), to_np(w))
            assert float((got - ref).abs().max()) <= 2 * tol
    assert torch.equal(kc[:, :p], kc0[:, :p]) and torch.equal(kc[:, p + sk:], kc0[:, p + sk:])
    assert torch.equal(vc[:, :p], vc0[:, :p]) and torch.equal(vc[:, p + sk:], vc0[:, p + sk:])
    q = gh.linear(q_in.reshape(b * sq, e), wq, bq).reshape(b, sq, e)
    attn = gh.ops.kv_attention(q, kc, vc, p + sk, h)
    ref = gh.linear(attn.reshape(b * sq, e), wo, bo).reshape(b, sq, e)
    if exact:
        assert torch.equal(out, ref)
    else:
        assert_rel(to_np(out), to_np(ref).astype(np.float64))
