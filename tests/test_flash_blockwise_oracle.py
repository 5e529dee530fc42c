"""Pins the oracle's restatement of FlashAttention::forward
(ghostflow-nn/src/flash_attention.rs:81-250), gfo_flash_attention_blockwise,
without running the reference (Rust; no toolchain here):

* a case worked out by hand from the reference loop: equal scores, v =
  3, 6, 9, block_n = 2 gives 5 -- (6 + 9) / 3, because the correction
  exp(old_max - new_max) multiplies the output once per KEY
  (:233-241), so the first block (correction exp(-inf) = 0) keeps only its
  last key;
* block_n = 1: one key per block makes the recurrence the exact online
  softmax, so the output must equal fp64 softmax attention (non-causal, and
  causal with top-left absolute indices j <= i for sq != sk both ways) and
  the ops.rs flash_attention oracle at sq == sk;
* an fp64 closed form of the same recurrence, written as one weight per key
  (log-weight s_j - m_t + (n_t - 1 - idx) (m_{t-1} - m_t) + the sum over
  later blocks of n_t' (m_{t'-1} - m_t'), divided by sum_j exp(s_j - m_last))
  -- a different algebra from the loop, so a dropped term, a wrong power or
  an off-by-one block boundary in either fails the comparison;
* derived properties: one block keeps p_last v_last / sum p; causal rows
  below block_n - 1 of the first query block are exactly 0 (their block's
  last key is masked); no keys gives zeros; a zero block size is an error.
Test infrastructure only (CPU)."""
import math

import numpy as np
import pytest

from _util import assert_rel


def _O():
    from oracle import oracle
    return oracle


def _data(bsz, sq, sk, d, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((bsz, sq, d)).astype(np.float32),
            rng.standard_normal((bsz, sk, d)).astype(np.float32),
            rng.standard_normal((bsz, sk, d)).astype(np.float32))


def _fp64_attention(q, k, v, scale, causal):
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * scale
    if causal:
        i = np.arange(q.shape[1])[:, None]
        j = np.arange(k.shape[1])[None, :]
        s = np.where(j <= i, s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    e = np.exp(s)
    return np.einsum("bij,bjd->bid", e / e.sum(-1, keepdims=True), v.astype(np.float64))


def _closed_form(q, k, v, bm, bn, causal, scale):
    """fp64 weights of the reference recurrence, one per key."""
    bsz, sq, d = q.shape
    sk = k.shape[1]
    out = np.zeros((bsz, sq, d))
    for b in range(bsz):
        s = (q[b].astype(np.float64) @ k[b].astype(np.float64).T) * float(np.float32(scale))
        for i in range(sq):
            end_i = min((i // bm + 1) * bm, sq)
            blocks = [(j0, min(j0 + bn, sk)) for j0 in range(0, sk, bn) if not (causal and j0 >= end_i)]
            if not blocks:
                continue
            vis = [(not causal) or j <= i for j in range(sk)]
            ms, m = [], -math.inf
            for j0, j1 in blocks:
                bmax = max((s[i, j] for j in range(j0, j1) if vis[j]), default=-math.inf)
                m = max(m, bmax)
                ms.append(m)
            l = sum(math.exp(s[i, j] - ms[-1]) for j0, j1 in blocks for j in range(j0, j1) if vis[j])
            delta = [0.0] + [ms[t - 1] - ms[t] for t in range(1, len(blocks))]
            ntail = [0.0] * len(blocks)  # sum over later blocks of n_t' * delta_t'
            for t in range(len(blocks) - 2, -1, -1):
                ntail[t] = ntail[t + 1] + (blocks[t + 1][1] - blocks[t + 1][0]) * delta[t + 1]
            acc = np.zeros(d)
            for t, (j0, j1) in enumerate(blocks):
                n = j1 - j0
                for j in range(j0, j1):
                    if not vis[j]:
                        continue
                    idx = j - j0
                    if t == 0:
                        if idx != n - 1:
                            continue  # multiplied by exp(-inf)^(n - 1 - idx) = 0
                        lw = s[i, j] - ms[0] + ntail[0]
                    else:
                        lw = s[i, j] - ms[t] + (n - 1 - idx) * delta[t] + ntail[t]
                    acc += math.exp(lw) * v[b, j].astype(np.float64)
            out[b, i] = acc / l if l > 0 else acc
    return out


def test_hand_derived_equal_scores():
    """q = 0 gives equal scores: block 0 (keys 0, 1) leaves o = v1 = 6 with
    row_sum 2; block 1 (key 2, correction exp(0) = 1) gives o = 15, row_sum
    3; the output is 5 (softmax attention would give 6)."""
    O = _O()
    q = np.zeros((1, 1, 1), np.float32)
    k = np.zeros((1, 3, 1), np.float32)
    v = np.array([[[3.0], [6.0], [9.0]]], np.float32)
    assert O.flash_attention_blockwise(q, k, v, 64, 2, False, 1.0).item() == 5.0
    assert O.flash_attention_blockwise(q, k, v, 64, 1, False, 1.0).item() == 6.0
    assert O.flash_attention_blockwise(q, k, v, 64, 3, False, 1.0).item() == 3.0  # one block: v2 / 3


@pytest.mark.parametrize("sq,sk,causal", [(9, 9, False), (9, 9, True), (6, 11, True), (11, 6, True),
                                          (5, 13, False)])
def test_block_n_one_is_softmax_attention(sq, sk, causal):
    O = _O()
    q, k, v = _data(2, sq, sk, 8, sq * 100 + sk)
    got = O.flash_attention_blockwise(q, k, v, 4, 1, causal, 0.3)
    assert_rel(got, _fp64_attention(q, k, v, np.float32(0.3), causal), tol=2e-6)


def test_block_n_one_matches_ops_flash_attention():
    """At sq == sk the reference's GPU-API twin (ops.rs:166-224, causal
    j > i) and FlashAttention with one key per block are the same
    attention."""
    O = _O()
    q, k, v = _data(3, 17, 17, 16, 5)
    scale = np.float32(1.0) / np.sqrt(np.float32(16))
    for causal in (False, True):
        got = O.flash_attention_blockwise(q, k, v, 5, 1, causal, scale)
        assert_rel(got, O.flash_attention(q, k, v, scale, causal))


@pytest.mark.parametrize("bm,bn,sq,sk,causal", [(64, 64, 20, 20, False), (4, 8, 21, 37, False),
                                                (4, 8, 21, 37, True), (8, 4, 37, 21, True),
                                                (3, 5, 13, 13, True), (64, 16, 70, 70, True),
                                                (5, 7, 1, 30, False), (2, 3, 30, 1, True)])
def test_closed_form(bm, bn, sq, sk, causal):
    O = _O()
    q, k, v = _data(2, sq, sk, 6, bm * 31 + bn * 7 + sq + sk)
    got = O.flash_attention_blockwise(q, k, v, bm, bn, causal, 0.45)
    ref = _closed_form(q, k, v, bm, bn, causal, 0.45)
    assert_rel(got, ref, tol=2e-5)


def test_single_block_keeps_last_key():
    """block_n >= sk: one block, correction 0 for every key but the last, so
    row i is p_last v_last / sum_j p_j with p_j = exp(s_j - max)."""
    O = _O()
    q, k, v = _data(1, 7, 10, 4, 11)
    got = O.flash_attention_blockwise(q, k, v, 64, 64, False, 0.5)
    s = (q[0].astype(np.float64) @ k[0].astype(np.float64).T) * 0.5
    p = np.exp(s - s.max(1, keepdims=True))
    ref = (p[:, -1:] * v[0, -1].astype(np.float64)) / p.sum(1, keepdims=True)
    assert_rel(got[0], ref, tol=2e-6)


def test_causal_first_rows_are_zero():
    """Causal with the default blocks: for rows i < block_n - 1 of the first
    query block, the last key of block 0 is masked (score 0 after the
    exp), so the output is 0 after block 0 and later blocks are fully
    masked (correction 1): the output is exactly 0."""
    O = _O()
    q, k, v = _data(2, 80, 80, 8, 3)
    got = O.flash_attention_blockwise(q, k, v, 64, 64, True, 0.35)
    assert (got[:, :63] == 0.0).all()
    assert (got[:, 63:] != 0.0).any(axis=-1).all()


def test_edge_cases():
    O = _O()
    q, k, v = _data(2, 4, 0, 3, 1)
    assert (O.flash_attention_blockwise(q, k, v, 64, 64, True, 1.0) == 0.0).all()
    q, k, v = _data(1, 4, 4, 3, 1)
    with pytest.raises(ValueError):
        O.flash_attention_blockwise(q, k, v, 0, 64, False, 1.0)
    with pytest.raises(ValueError):
        O.flash_attention_blockwise(q, k, v, 64, 0, False, 1.0)


def test_reference_unit_test_shapes():
    """flash_attention.rs:312-340: [2, 8, 16] with the default config and
    [1, 4, 8] with FlashAttentionConfig::causal(1.0) keep their shapes."""
    O = _O()
    q, k, v = _data(2, 8, 8, 16, 0)
    assert O.flash_attention_blockwise(q, k, v, 64, 64, False, 1.0).shape == (2, 8, 16)
    q, k, v = _data(1, 4, 4, 8, 0)
    assert O.flash_attention_blockwise(q, k, v, 64, 64, True, 1.0).shape == (1, 4, 8)


@pytest.mark.parametrize("bm,bn,sq,sk,causal", [(64, 64, 20, 20, False), (4, 8, 21, 37, False),
                                                (4, 8, 21, 37, True), (8, 4, 37, 21, True),
                                                (3, 5, 13, 13, True), (64, 16, 70, 70, True),
                                                (5, 7, 1, 30, False), (2, 3, 30, 1, True),
                                                (16, 1, 9, 40, False), (7, 5, 29, 31, True)])
def test_vectorized_closed_form(bm, bn, sq, sk, causal):
    """The vectorized fp64 closed form the GPU tests use as the exact value
    agrees with the per-row loop above (itself pinned against the oracle)."""
    from _flash_exact import flash_blockwise_exact
    q, k, v = _data(2, sq, sk, 6, bm * 13 + bn * 5 + sq + sk)
    a = flash_blockwise_exact(q, k, v, bm, bn, causal, 0.45)
    b = _closed_form(q, k, v, bm, bn, causal, 0.45)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-14)
