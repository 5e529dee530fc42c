"""The reference's quantization types on this library
(ghostflow-nn/src/quantization.rs), with the codes, scales and zero points
computed on the device by the bit-exact kernels of quant.hip:

  QuantizationScheme          :11-18   INT8, FP16, Dynamic
  QuantizationConfig          :22-37   default INT8, per channel, symmetric
  QuantizedTensor             :40-214  from_tensor, dequantize, compression_ratio
  QuantizationAwareTraining   :219-247 fake_quantize = dequantize(from_tensor)
  DynamicQuantization         :251-294 per-channel symmetric weights,
                                       per-tensor asymmetric activations

DynamicQuantization.quantized_linear runs the INT8 linear on its stored
weights and a dynamically quantized activation (gfh_qlinear_dynamic_i8:
quantize_activation then gfh_qlinear_i8, one launch at decode sizes) -- the
layer the reference only expresses as get_weights + fp32 matmul.  FP16 raises NotImplementedError, as the reference's
unimplemented!() does (quantization.rs:155-158, :167-168).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass

import torch

from . import _lib
from .ops import (GhostFlowError, dequantize, qlinear_dynamic, quantize_per_channel, quantize_per_tensor,
                  qweight_rowsum)


class QuantizationScheme(enum.IntEnum):
    """quantization.rs:11-18 (the GHOSTFLQ file records this value)."""
    INT8 = 0
    FP16 = 1
    Dynamic = 2


@dataclass
class QuantizationConfig:
    """quantization.rs:22-37."""
    scheme: QuantizationScheme = QuantizationScheme.INT8
    per_channel: bool = True
    symmetric: bool = True


class QuantizedTensor:
    """quantization.rs:40-51: int8 codes of `shape`, one scale and zero point
    per channel (dim 0) or one for the whole tensor, on the device."""

    def __init__(self, data, scales, zero_points, shape, scheme=QuantizationScheme.INT8):
        self.data = data
        self.scales = scales
        self.zero_points = zero_points
        self.shape = tuple(shape)
        self.scheme = QuantizationScheme(scheme)

    @classmethod
    def from_tensor(cls, tensor, config: QuantizationConfig | None = None) -> "QuantizedTensor":
        """quantization.rs:55-75: per channel over dim 0 or per tensor; the
        reference reads the raw storage, so the tensor must be contiguous."""
        config = config or QuantizationConfig()
        if config.scheme == QuantizationScheme.FP16:
            raise NotImplementedError("FP16 quantization requires half-precision support")
        if tensor.dim() == 0:
            raise GhostFlowError(_lib.INVALID_SHAPE, "quantization needs at least one dimension")
        if config.per_channel:
            q, s, z = quantize_per_channel(tensor, symmetric=config.symmetric)
        else:
            q, s, z = quantize_per_tensor(tensor, symmetric=config.symmetric)
        return cls(q, s, z, tensor.shape, QuantizationScheme.INT8)

    def dequantize(self):
        """quantization.rs:162-204: (q - zp) * scale, per tensor when there is
        one scale, else per row."""
        if self.scheme == QuantizationScheme.FP16:
            raise NotImplementedError("FP16 dequantization not yet implemented")
        return dequantize(self.data, self.scales, self.zero_points).reshape(self.shape)

    def compression_ratio(self) -> float:
        """quantization.rs:207-213."""
        n = self.data.numel()
        return (n * 4) / (n + self.scales.numel() * 4 + self.zero_points.numel())


class QuantizationAwareTraining:
    """quantization.rs:219-247."""

    def __init__(self, config: QuantizationConfig | None = None):
        self.config = config or QuantizationConfig()
        self.fake_quantize_enabled = True

    def fake_quantize(self, tensor):
        if not self.fake_quantize_enabled:
            return tensor.clone()
        return QuantizedTensor.from_tensor(tensor, self.config).dequantize()

    def set_fake_quantize(self, enabled: bool) -> None:
        self.fake_quantize_enabled = bool(enabled)


class DynamicQuantization:
    """quantization.rs:251-294: weights quantized once per channel,
    symmetric; activations per tensor, asymmetric, at run time."""

    def __init__(self):
        self.config = QuantizationConfig(QuantizationScheme.Dynamic, per_channel=True, symmetric=True)
        self.weight_quantized: dict[str, QuantizedTensor] = {}
        self._rowsums: dict[str, torch.Tensor] = {}

    def quantize_weights(self, name: str, weights) -> None:
        # the Dynamic scheme quantizes as INT8 and records INT8 (quantization.rs:59, :150)
        q = QuantizedTensor.from_tensor(weights, self.config)
        self.weight_quantized[name] = q
        if weights.dim() == 2:
            self._rowsums[name] = qweight_rowsum(q.data)

    def get_weights(self, name: str):
        q = self.weight_quantized.get(name)
        return None if q is None else q.dequantize()

    def quantize_activation(self, activation) -> QuantizedTensor:
        return QuantizedTensor.from_tensor(
            activation, QuantizationConfig(QuantizationScheme.INT8, per_channel=False, symmetric=False))

    def quantized_linear(self, name: str, x, bias=None):
        """y = x . W^T (+ bias) as the INT8 linear: x [m, in] quantized per
        tensor (asymmetric), the stored weight [out, in] per channel;
        acc = sum (qx - zx) qw exactly in int32, y = acc * (sx * sw) + bias."""
        q = self.weight_quantized[name]
        if len(q.shape) != 2:
            raise GhostFlowError(_lib.INVALID_SHAPE, f"{name} is not a [out, in] weight")
        y = qlinear_dynamic(x.reshape(-1, x.shape[-1]).contiguous(), q.data, q.scales, self._rowsums[name],
                            bias=bias)
        return y.reshape(*x.shape[:-1], q.shape[0])
