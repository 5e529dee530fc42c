"""Module-level mirrors of the reference's attention and feed-forward layers.

MultiHeadAttention follows ghostflow-nn/src/attention.rs:66-170: four
embed_dim x embed_dim Linear projections stored [out, in] with biases,
forward_with_cache(query, key, value, mask, past_key, past_value) ->
(output, attn_weights, k_cache, v_cache), and forward(input) as
self-attention.  Dropout is not implemented on this path: in training mode
with dropout > 0 (the reference's default mode is training) the calls
raise, so use eval() or dropout 0.

KVCache is the in-place form of the reference's past_key / past_value
concatenation: preallocated [B, capacity, E] buffers that every step
appends to, so a decode step costs no copy of the past.

SwiGLU follows ghostflow-nn/src/llama.rs:259-287 (LLaMA / Mistral
feed-forward); QuantizedSwiGLU is the same block with DynamicQuantization's
int8 weights (ghostflow-nn/src/quantization.rs:251-288).
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .ops import (GhostFlowError, flash_attention_blockwise, mha_forward_cached, mha_forward_with_cache, qswiglu,
                  quantize_per_channel, qweight_rowsum, swiglu)


class FlashAttentionConfig:
    """FlashAttentionConfig (ghostflow-nn/src/flash_attention.rs:14-68):
    block sizes, causal flag, dropout (stored, never applied by the
    reference's forward) and scale (default 1.0, not 1/sqrt(d))."""

    def __init__(self, block_size_m=64, block_size_n=64, causal=False, dropout=0.0, scale=1.0):
        self.block_size_m = block_size_m
        self.block_size_n = block_size_n
        self.causal = causal
        self.dropout = dropout
        self.scale = scale

    @classmethod
    def causal_config(cls, scale):
        """FlashAttentionConfig::causal(scale) (:41-47)."""
        return cls(causal=True, scale=scale)

    @classmethod
    def bidirectional(cls, scale):
        """FlashAttentionConfig::bidirectional(scale) (:50-56)."""
        return cls(causal=False, scale=scale)

    @classmethod
    def long_sequence(cls, scale):
        """FlashAttentionConfig::long_sequence(scale) (:59-66): 128 x 128 blocks."""
        return cls(block_size_m=128, block_size_n=128, scale=scale)


class FlashAttention:
    """FlashAttention (flash_attention.rs:70-296): forward(query, key, value)
    on [batch, seq_len, d_model] device tensors, the reference's blockwise
    recurrence on the GPU (gfh_flash_attention_f32)."""

    def __init__(self, config: FlashAttentionConfig | None = None):
        self.config = config or FlashAttentionConfig()

    def forward(self, query, key, value):
        c = self.config
        return flash_attention_blockwise(query, key, value, block_size_m=c.block_size_m,
                                         block_size_n=c.block_size_n, causal=c.causal, scale=c.scale)

    __call__ = forward

    def memory_usage_ratio(self, seq_len: int, _d_model: int) -> float:
        """(block_m * block_n) / seq_len^2, as the reference reports (:285-295)."""
        return float(self.config.block_size_m * self.config.block_size_n) / float(seq_len * seq_len)


class KVCache:
    """Keys and values of the positions seen so far, [B, capacity, E]."""

    def __init__(self, batch: int, capacity: int, embed_dim: int, device="cuda"):
        self.k = torch.empty((batch, capacity, embed_dim), dtype=torch.float32, device=device)
        self.v = torch.empty_like(self.k)
        self.length = 0

    @property
    def capacity(self) -> int:
        return self.k.shape[1]

    def reset(self) -> None:
        self.length = 0


class MultiHeadAttention:
    """ghostflow-nn MultiHeadAttention (attention.rs:66-170) on the GPU."""

    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, device="cuda"):
        if embed_dim % num_heads:
            raise GhostFlowError(_lib.INVALID_SHAPE, "embed_dim must be divisible by num_heads")
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.dropout_p = dropout
        self.training = True
        # Linear::new's init (ghostflow-nn/src/linear.rs:23-33, init.rs:31-41):
        # W ~ U(+-sqrt(6/in)), b ~ U(+-1/sqrt(in)); the reference draws from
        # an unseeded RNG, so only the distribution is kept.
        wb, bb = math.sqrt(6.0 / embed_dim), 1.0 / math.sqrt(embed_dim)
        mk = lambda shape, bound: (torch.rand(shape, device=device) * 2 - 1) * bound  # noqa: E731
        self.q_weight, self.k_weight, self.v_weight, self.out_weight = (
            mk((embed_dim, embed_dim), wb) for _ in range(4))
        self.q_bias, self.k_bias, self.v_bias, self.out_bias = (mk((embed_dim,), bb) for _ in range(4))

    def _weights(self):
        if self.training and self.dropout_p > 0:
            raise GhostFlowError(_lib.INVALID_DATA, "attention dropout is not implemented on this path; "
                                 "call eval() or use dropout 0")
        return (self.q_weight, self.q_bias, self.k_weight, self.k_bias, self.v_weight, self.v_bias,
                self.out_weight, self.out_bias)

    def forward_with_cache(self, query, key, value, mask=None, past_key=None, past_value=None):
        return mha_forward_with_cache(query, key, value, *self._weights(), self.num_heads, mask=mask,
                                      past_key=past_key, past_value=past_value)

    def forward(self, x):
        return self.forward_with_cache(x, x, x)[0]

    __call__ = forward

    def step(self, x, cache: KVCache, *, mask=None, causal=False, want_weights=False):
        """Self-attention of x [B, S, E] (new positions) over the cache plus
        x, appending x's keys and values to the cache in place."""
        s = x.shape[1]
        if cache.length + s > cache.capacity:
            raise GhostFlowError(_lib.INVALID_SHAPE, "KV cache is full")
        r = mha_forward_cached(x, x, x, *self._weights(), self.num_heads, cache.k, cache.v, cache.length,
                               mask=mask, causal=causal, want_weights=want_weights)
        cache.length += s
        return r

    def parameters(self):
        return [self.q_weight, self.q_bias, self.k_weight, self.k_bias, self.v_weight, self.v_bias,
                self.out_weight, self.out_bias]

    def train(self):
        self.training = True

    def eval(self):
        self.training = False

    def is_training(self) -> bool:
        return self.training


class SwiGLU:
    """ghostflow-nn SwiGLU (llama.rs:259-287): gate_proj and up_proj
    Linear(hidden, inter), down_proj Linear(inter, hidden), all with bias
    (Linear::new), forward = down(silu(gate(x)) * up(x)) on the GPU."""

    def __init__(self, hidden_size: int, intermediate_size: int, device="cuda"):
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size

        # Linear::new's init (linear.rs:23-33, init.rs:31-41) with an unseeded
        # RNG in the reference, so only the distribution is kept.
        def lin(n_in, n_out):
            wb, bb = math.sqrt(6.0 / n_in), 1.0 / math.sqrt(n_in)
            w = (torch.rand((n_out, n_in), device=device) * 2 - 1) * wb
            b = (torch.rand((n_out,), device=device) * 2 - 1) * bb
            return w, b

        self.gate_weight, self.gate_bias = lin(hidden_size, intermediate_size)
        self.up_weight, self.up_bias = lin(hidden_size, intermediate_size)
        self.down_weight, self.down_bias = lin(intermediate_size, hidden_size)

    def forward(self, x):
        """x [..., hidden] -> [..., hidden]."""
        lead = x.shape[:-1]
        y = swiglu(x.reshape(-1, self.hidden_size).contiguous(), self.gate_weight, self.gate_bias,
                   self.up_weight, self.up_bias, self.down_weight, self.down_bias)
        return y.reshape(*lead, self.hidden_size)

    __call__ = forward

    def parameters(self):
        return [self.gate_weight, self.gate_bias, self.up_weight, self.up_bias, self.down_weight,
                self.down_bias]

    def quantize(self) -> "QuantizedSwiGLU":
        """DynamicQuantization of each projection (quantization.rs:251-288):
        weights per-channel symmetric int8, biases kept in fp32."""
        return QuantizedSwiGLU(self)


class QuantizedSwiGLU:
    """SwiGLU with DynamicQuantization's int8 weights: codes [out, in],
    per-row scales, per-row code sums for the activation zero point.
    Activations are quantized per tensor (asymmetric) on each call."""

    def __init__(self, layer: SwiGLU):
        self.hidden_size = layer.hidden_size
        self.intermediate_size = layer.intermediate_size

        def q(w, b):
            codes, scales, _zp = quantize_per_channel(w, symmetric=True)
            return codes, scales, qweight_rowsum(codes), b

        self.gate = q(layer.gate_weight, layer.gate_bias)
        self.up = q(layer.up_weight, layer.up_bias)
        self.down = q(layer.down_weight, layer.down_bias)

    def forward(self, x):
        lead = x.shape[:-1]
        y = qswiglu(x.reshape(-1, self.hidden_size).contiguous(), self.gate, self.up, self.down)
        return y.reshape(*lead, self.hidden_size)

    __call__ = forward
