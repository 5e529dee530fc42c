"""FlashAttention::forward (ghostflow-nn/src/flash_attention.rs:81-250) on
the GPU (gfh_flash_attention_f32) against the oracle's restatement of the
same blockwise recurrence (gfo_flash_attention_blockwise), on [batch,
seq_len, d_model] inputs with FlashAttentionConfig's block sizes, causal
flag and scale.

Bar, per element: |gpu - exact| <= 2 |oracle - exact| + 1e-4 mean|oracle|,
where `exact` is the fp64 closed form of the same recurrence
(_flash_exact.flash_blockwise_exact, pinned against the per-row loop and
the oracle on the CPU).  The reference's own fp32 evaluation strays from
the exact value (this recurrence concentrates its weight on few keys and
its outputs are small), so the GPU may stray as far, twice over, plus the
north star's 1e-4 relative to the output's scale; every element the
reference leaves at exactly 0 must be exactly 0, and normwise max|gpu -
oracle| <= 1e-4 max|oracle| as well."""
import numpy as np
import pytest

from _util import assert_rel, to_dev, to_np


def _check(got, ref, tol=1e-4):
    np.testing.assert_array_equal(got == 0.0, ref == 0.0)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    assert err <= tol * float(np.abs(ref).max()), (err, float(np.abs(ref).max()))


def _check_exact(got, ref, exact, tol=1e-4):
    """Per element against the fp64 closed form (module docstring)."""
    _check(got, ref, tol)
    e_gpu = np.abs(got.astype(np.float64) - exact)
    e_ref = np.abs(ref.astype(np.float64) - exact)
    bound = 2.0 * e_ref + tol * float(np.abs(ref).mean())
    bad = e_gpu > bound
    assert not bad.any(), (int(bad.sum()), float(e_gpu[bad].max()), float(bound[bad].min()))

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _O():
    from oracle import oracle
    return oracle


def _inputs(bsz, sq, sk, d, seed):
    from ghostflow_hip import synth
    return (synth.normal((bsz, sq, d), seed=seed, tensor_id=0), synth.normal((bsz, sk, d), seed=seed, tensor_id=1),
            synth.normal((bsz, sk, d), seed=seed, tensor_id=2))


CASES = [
    # (batch, sq, sk, d, block_m, block_n, causal, scale)
    (2, 8, 8, 16, 64, 64, False, 1.0),          # the reference's unit-test shape, default config
    (1, 4, 4, 8, 64, 64, True, 1.0),            # FlashAttentionConfig::causal(1.0) unit test
    (2, 200, 200, 64, 64, 64, True, 0.125),     # several query / key blocks, causal
    (2, 150, 333, 32, 64, 64, True, 0.18),      # sq < sk: top-left causal
    (3, 333, 150, 32, 64, 64, True, 0.18),      # sq > sk: rows past sk see every key
    (2, 257, 300, 48, 128, 128, False, 0.14),   # FlashAttentionConfig::long_sequence
    (2, 97, 101, 40, 7, 5, True, 0.16),         # odd block sizes, ragged last blocks
    (1, 64, 700, 20, 16, 1, False, 0.22),       # block_n = 1: softmax attention, 700 blocks
    (20, 33, 65, 37, 64, 64, True, 0.16),       # d % 4 != 0, many batches (strided-batched GEMMs)
    (4, 512, 512, 128, 64, 64, True, 0.0883883476),
    # the fused two-pass form (block_n a multiple of 32, d % 4 == 0, d <= 128)
    (3, 130, 130, 128, 64, 32, True, 0.09),     # one 32-key tile per block
    (2, 300, 290, 64, 48, 96, True, 0.12),      # three tiles per block, ragged last block
    (2, 181, 250, 128, 64, 64, False, 0.09),    # non-causal, ragged key blocks
    (2, 40, 20, 16, 64, 64, True, 0.3),         # every key in block 0 (sk < block_n)
    (1, 2048, 2048, 128, 64, 64, True, 0.0883883476),  # the bench's sequence length
    (1, 4096, 4096, 128, 64, 64, True, 0.0883883476),  # 64 key blocks for the heaviest query sets
    (2, 77, 333, 128, 128, 256, True, 0.09),    # block_n larger than a workgroup's queries
]


@pytest.mark.parametrize("bsz,sq,sk,d,bm,bn,causal,scale", CASES)
def test_flash_attention_vs_oracle(torch_dev, bsz, sq, sk, d, bm, bn, causal, scale):
    gh, O = _gh(), _O()
    q, k, v = _inputs(bsz, sq, sk, d, bsz * 1000 + sq + sk + d)
    from _flash_exact import flash_blockwise_exact
    ref = O.flash_attention_blockwise(q, k, v, bm, bn, causal, scale)
    got = to_np(gh.flash_attention_blockwise(to_dev(q, torch_dev), to_dev(k, torch_dev), to_dev(v, torch_dev),
                                             block_size_m=bm, block_size_n=bn, causal=causal, scale=scale))
    _check_exact(got, ref, flash_blockwise_exact(q, k, v, bm, bn, causal, scale))


def test_fused_and_three_step_forms_agree(torch_dev):
    """The same layer through both GPU forms: block_n = 64 takes the fused
    two-pass kernel on aligned inputs and the scores / weights / weights.V
    path when q starts 4 bytes into its buffer (not 16-byte aligned)."""
    import torch
    gh = _gh()
    q, k, v = _inputs(2, 200, 260, 64, 77)
    dq, dk, dv = (to_dev(a, torch_dev) for a in (q, k, v))
    fused = to_np(gh.flash_attention_blockwise(dq, dk, dv, block_size_m=64, block_size_n=64, causal=True,
                                               scale=0.125))
    buf = torch.empty(dq.numel() + 1, device=torch_dev)
    dq_off = buf[1:].view_as(dq)
    dq_off.copy_(dq)
    three = to_np(gh.flash_attention_blockwise(dq_off, dk, dv, block_size_m=64, block_size_n=64, causal=True,
                                               scale=0.125))
    np.testing.assert_array_equal(fused == 0.0, three == 0.0)
    assert float(np.abs(fused - three).max()) <= 1e-4 * float(np.abs(three).max())


def test_block_n_one_is_sdpa(torch_dev):
    """One key per block: the reference recurrence is exact softmax
    attention, so the GPU layer equals the fused SDPA kernel on [B, 1, S, d]
    within the bar."""
    gh = _gh()
    q, k, v = _inputs(2, 96, 96, 64, 9)
    dq, dk, dv = (to_dev(a, torch_dev) for a in (q, k, v))
    got = to_np(gh.flash_attention_blockwise(dq, dk, dv, block_size_m=32, block_size_n=1, causal=True, scale=0.125))
    sd = to_np(gh.sdpa(dq[:, None], dk[:, None], dv[:, None], scale=0.125, causal=True))[:, 0]
    assert_rel(got, sd)


def test_module_api_and_errors(torch_dev):
    """FlashAttention(FlashAttentionConfig) forward, the reference's Err
    cases (non-3-D inputs, a d_model mismatch), a zero block size, no keys
    (zeros) and a caller workspace."""
    import torch
    gh, O = _gh(), _O()
    q, k, v = _inputs(2, 10, 12, 8, 4)
    dq, dk, dv = (to_dev(a, torch_dev) for a in (q, k, v))
    fa = gh.FlashAttention(gh.FlashAttentionConfig(block_size_m=4, block_size_n=3, causal=True, scale=0.5))
    _check(to_np(fa.forward(dq, dk, dv)), O.flash_attention_blockwise(q, k, v, 4, 3, True, 0.5))
    with pytest.raises(gh.GhostFlowError, match="Expected 3D"):
        fa.forward(dq[0], dk, dv)
    with pytest.raises(gh.GhostFlowError, match="same d_model"):
        fa.forward(dq, dk[..., :4].contiguous(), dv)
    with pytest.raises(gh.GhostFlowError, match="block sizes"):
        gh.flash_attention_blockwise(dq, dk, dv, block_size_m=0)
    empty = torch.empty((2, 0, 8), device=torch_dev)
    out = gh.flash_attention_blockwise(dq, empty, empty)
    assert bool((out == 0).all())
    ws = torch.empty(int(gh.lib().gfh_flash_attention_workspace_size(2, 10, 12)) // 4, device=torch_dev)
    got = gh.flash_attention_blockwise(dq, dk, dv, block_size_m=4, block_size_n=3, causal=True, scale=0.5,
                                       workspace=ws)
    np.testing.assert_array_equal(to_np(got), to_np(fa.forward(dq, dk, dv)))


def test_workspace_bytes_counted_by_dtype(torch_dev):
    """A caller workspace is measured in bytes whatever its dtype: a uint8
    workspace of exactly the queried size works; one byte short is rejected
    with InvalidShape before any launch."""
    import torch
    gh = _gh()
    q, k, v = _inputs(2, 10, 12, 8, 4)
    dq, dk, dv = (to_dev(a, torch_dev) for a in (q, k, v))
    need = int(gh.lib().gfh_flash_attention_workspace_size(2, 10, 12))
    assert need > 0
    kw = dict(block_size_m=4, block_size_n=3, causal=True, scale=0.5)
    want = to_np(gh.flash_attention_blockwise(dq, dk, dv, **kw))
    ws = torch.empty(need, dtype=torch.uint8, device=torch_dev)
    np.testing.assert_array_equal(to_np(gh.flash_attention_blockwise(dq, dk, dv, workspace=ws, **kw)), want)
    short = torch.empty(need - 1, dtype=torch.uint8, device=torch_dev)
    with pytest.raises(gh.GhostFlowError) as ei:
        gh.flash_attention_blockwise(dq, dk, dv, workspace=short, **kw)
    assert ei.value.status == 1


def test_too_many_key_blocks_rejected(torch_dev):
    import torch
    gh = _gh()
    q = torch.zeros((1, 2, 4), device=torch_dev)
    k = torch.zeros((1, 8193, 4), device=torch_dev)
    with pytest.raises(gh.GhostFlowError, match="key blocks"):
        gh.flash_attention_blockwise(q, k, k, block_size_n=1)
