"""fp64 closed form of FlashAttention::forward's blockwise recurrence
(ghostflow-nn/src/flash_attention.rs:137-250), vectorized over query rows.

For query row i, key block t (keys j0_t .. j0_t + n_t - 1, processed only
while t < T_i: causal skips every block with j0_t >= the end of i's query
block), running max m_t after block t and delta_t = m_{t-1} - m_t
(delta_0 = -inf), the recurrence multiplies the output by
exp(delta_t) once per KEY of block t and the running sum once per block.
So key j = j0_t + idx, visible to row i, ends with the weight

    exp(s_ij - m_t + (n_t - 1 - idx) delta_t + sum_{t < t' < T_i} n_t' delta_t')

(in block 0 only the last key survives: exp(-inf)^(n_0 - 1 - idx)), and the
output is sum_j weight_j v_j / sum_{visible j} exp(s_ij - m_last).  The
per-row loop of the same algebra, pinned against the oracle, is
_closed_form in test_flash_blockwise_oracle.py; this module is checked
against it there."""
import numpy as np


def flash_blockwise_exact(q, k, v, bm, bn, causal, scale):
    """q [B, Sq, d], k / v [B, Sk, d] -> fp64 [B, Sq, d]."""
    bsz, sq, d = q.shape
    sk = k.shape[1]
    out = np.zeros((bsz, sq, d))
    if sk == 0 or sq == 0:
        return out
    nb = -(-sk // bn)
    pad = nb * bn - sk
    i = np.arange(sq)
    j = np.arange(sk)
    tj = j // bn                                    # block of key j
    idx = j - tj * bn                               # position in its block
    n_t = np.minimum(bn, sk - np.arange(nb) * bn)   # keys per block
    if causal:
        end_i = np.minimum((i // bm + 1) * bm, sq)
        T = np.minimum(-(-end_i // bn), nb)         # blocks row i processes
        vis = j[None, :] <= i[:, None]
    else:
        T = np.full(sq, nb)
        vis = np.ones((sq, sk), bool)
    live_t = np.arange(nb)[None, :] < T[:, None]    # [sq, nb]
    vis = vis & live_t[:, tj]
    sc = float(np.float32(scale))
    for b in range(bsz):
        s = (q[b].astype(np.float64) @ k[b].astype(np.float64).T) * sc
        sm = np.where(vis, s, -np.inf)
        bmax = np.pad(sm, ((0, 0), (0, pad)), constant_values=-np.inf).reshape(sq, nb, bn).max(-1)
        m = np.maximum.accumulate(bmax, axis=1)     # running max after each block
        m_last = m[i, T - 1]
        delta = np.full((sq, nb), -np.inf)
        delta[:, 1:] = m[:, :-1] - m[:, 1:]
        nd = np.where(live_t, n_t[None, :] * np.where(np.isfinite(delta), delta, 0.0), 0.0)
        nd[:, 0] = 0.0
        # ntail[t] = sum over t < t' < T of n_t' delta_t'
        ntail = np.cumsum(nd[:, ::-1], axis=1)[:, ::-1] - nd
        rest = (n_t[tj] - 1 - idx)[None, :]
        d_j = delta[:, tj]
        with np.errstate(invalid="ignore"):
            pw = np.where(tj[None, :] == 0, np.where(rest == 0, 0.0, -np.inf), rest * d_j)
        lw = s - m[:, tj] + pw + ntail[:, tj]
        w = np.where(vis, np.exp(np.where(vis, lw, -np.inf)), 0.0)
        l_sum = np.where(vis, np.exp(np.where(vis, s - m_last[:, None], -np.inf)), 0.0).sum(1)
        o = w @ v[b].astype(np.float64)
        out[b] = np.where(l_sum[:, None] > 0, o / np.where(l_sum > 0, l_sum, 1.0)[:, None], o)
    return out
