"""The Python mirror of the reference's quantization types
(ghostflow-nn/src/quantization.rs) over the bit-exact device kernels:
defaults and FP16 behaviour on the CPU; codes, dequantized values, the
DynamicQuantization flow and the INT8 linear bit-exact against the oracle
on the GPU."""
import numpy as np
import pytest

from oracle import oracle as O
from _util import to_dev, to_np


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def test_config_defaults_and_fp16():
    gh = _gh()
    c = gh.QuantizationConfig()
    assert c.scheme == gh.QuantizationScheme.INT8 and c.per_channel and c.symmetric  # quantization.rs:28-37
    assert int(gh.QuantizationScheme.Dynamic) == 2
    with pytest.raises(NotImplementedError):
        gh.QuantizedTensor.from_tensor(None, gh.QuantizationConfig(gh.QuantizationScheme.FP16))
    dq = gh.DynamicQuantization()
    assert dq.config.scheme == gh.QuantizationScheme.Dynamic and dq.get_weights("missing") is None


@pytest.mark.gpu
@pytest.mark.parametrize("per_channel,symmetric", [(True, True), (True, False), (False, True), (False, False)])
def test_from_tensor_and_dequantize(torch_dev, per_channel, symmetric):
    gh = _gh()
    rng = np.random.default_rng(int(per_channel) * 2 + int(symmetric))
    x = rng.normal(0, 1, (37, 129)).astype(np.float32)
    qt = gh.QuantizedTensor.from_tensor(to_dev(x, torch_dev), gh.QuantizationConfig(per_channel=per_channel,
                                                                                      symmetric=symmetric))
    if per_channel:
        q, s, z = O.quantize_per_channel(x, symmetric)
    else:
        q, s, z = O.quantize_per_tensor(x, symmetric)
    np.testing.assert_array_equal(to_np(qt.data), q)
    np.testing.assert_array_equal(to_np(qt.scales).view(np.uint32), np.atleast_1d(s).view(np.uint32))
    np.testing.assert_array_equal(to_np(qt.zero_points), np.atleast_1d(z))
    assert qt.shape == (37, 129)
    np.testing.assert_array_equal(to_np(qt.dequantize()), O.dequantize(q, s, z))
    # compression_ratio (quantization.rs:207-213)
    n_s = 37 if per_channel else 1
    assert qt.compression_ratio() == pytest.approx(37 * 129 * 4 / (37 * 129 + 5 * n_s))
    # QAT fake quantization is the round trip
    qat = gh.QuantizationAwareTraining(gh.QuantizationConfig(per_channel=per_channel, symmetric=symmetric))
    np.testing.assert_array_equal(to_np(qat.fake_quantize(to_dev(x, torch_dev))), O.dequantize(q, s, z))
    qat.set_fake_quantize(False)
    np.testing.assert_array_equal(to_np(qat.fake_quantize(to_dev(x, torch_dev))), x)


@pytest.mark.gpu
def test_dynamic_quantization_flow(torch_dev):
    gh = _gh()
    rng = np.random.default_rng(7)
    w = (rng.normal(0, 0.02, (300, 256))).astype(np.float32)
    b = rng.uniform(-0.01, 0.01, 300).astype(np.float32)
    x = rng.normal(0, 1, (2, 5, 256)).astype(np.float32)
    dq = gh.DynamicQuantization()
    dq.quantize_weights("fc", to_dev(w, torch_dev))
    qw, sw, zw = O.quantize_per_channel(w, True)
    np.testing.assert_array_equal(to_np(dq.get_weights("fc")), O.dequantize(qw, sw, zw))
    xa = dq.quantize_activation(to_dev(x, torch_dev))
    qx, sx, zx = O.quantize_per_tensor(x, False)
    np.testing.assert_array_equal(to_np(xa.data), qx)
    y = to_np(dq.quantized_linear("fc", to_dev(x, torch_dev), bias=to_dev(b, torch_dev)))
    ref, _ = O.qlinear_i8(qx.reshape(10, 256), sx, zx, False, qw, sw, b, want_acc=False)
    assert y.shape == (2, 5, 300)
    np.testing.assert_array_equal(y.reshape(10, 300), ref)


@pytest.mark.gpu
def test_reference_unit_cases(torch_dev):
    """The cases of quantization.rs:299-430, through this API, with the
    reference's own tolerances and bit-exact against the oracle."""
    gh = _gh()
    Cfg, S = gh.QuantizationConfig, gh.QuantizationScheme
    cases = [  # (data, shape, config, tolerance)
        ([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], (2, 3), Cfg(S.INT8, False, True), 0.1),
        ([1.0, 2.0, 3.0, 10.0, 20.0, 30.0], (2, 3), Cfg(S.INT8, True, True), 0.5),
        ([-5.0, -3.0, -1.0, 1.0, 3.0, 5.0], (6,), Cfg(S.INT8, False, False), 0.1),
        ([1.0, 2.0, 3.0, 4.0], (4,), Cfg(), 0.1),
    ]
    for data, shape, cfg, tol in cases:
        x = np.array(data, np.float32).reshape(shape)
        qt = gh.QuantizedTensor.from_tensor(to_dev(x, torch_dev), cfg)
        back = to_np(qt.dequantize())
        assert back.shape == shape
        assert np.abs(back - x).max() < tol, (data, back)
        fn = O.quantize_per_channel if cfg.per_channel else O.quantize_per_tensor
        q, s, z = fn(x, cfg.symmetric)
        np.testing.assert_array_equal(to_np(qt.data), q)
        np.testing.assert_array_equal(back, O.dequantize(q, s, z))
    assert gh.QuantizedTensor.from_tensor(to_dev(np.array([[1, 2, 3], [10, 20, 30]], np.float32), torch_dev)
                                          ).scales.numel() == 2
    qt = gh.QuantizedTensor.from_tensor(to_dev(np.arange(1000, dtype=np.float32), torch_dev), Cfg(S.INT8, False, True))
    assert 3.5 < qt.compression_ratio() < 4.5
    dq = gh.DynamicQuantization()
    dq.quantize_weights("layer1", to_dev(np.array([[1, 2], [3, 4]], np.float32), torch_dev))
    assert tuple(dq.get_weights("layer1").shape) == (2, 2)
    qa = dq.quantize_activation(to_dev(np.array([0.5, 1.5, 2.5], np.float32), torch_dev))
    assert qa.shape == (3,) and qa.scales.numel() == 1
    # an N-d weight is quantized per dim-0 channel, like the reference's storage walk
    w3 = np.random.default_rng(3).normal(0, 1, (4, 5, 6)).astype(np.float32)
    q3 = gh.QuantizedTensor.from_tensor(to_dev(w3, torch_dev))
    qo, so, zo = O.quantize_per_channel(w3, True)
    np.testing.assert_array_equal(to_np(q3.data), qo)
    np.testing.assert_array_equal(to_np(q3.dequantize()), O.dequantize(qo, so, zo))
