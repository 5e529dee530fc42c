#!/usr/bin/env python3
"""Writes the golden fixtures in this directory from the CPU oracle.

Inputs come from the counter-based generator (ghostflow_hip.synth, seed 0
unless stated) or are the reference's own unit-test inputs; expected outputs
are the oracle's (oracle/gf_oracle.c, the restated reference CPU path).  Each
.npz holds plain arrays only (no pickled objects) plus a `meta` string naming
the generator, seeds, shapes and the reference function it exercises.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "ghost-flow_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from ghostflow_hip import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

GEMM_SHAPES = [(1, 1, 1), (7, 5, 3), (33, 17, 29), (64, 64, 64), (128, 96, 200)]


def gemm():
    out = {}
    for m, k, n in GEMM_SHAPES:
        a = synth.normal((m, k), seed=0, tensor_id=0)
        b = synth.normal((k, n), seed=0, tensor_id=1)
        tag = f"{m}x{k}x{n}"
        out[f"a_{tag}"], out[f"b_{tag}"], out[f"c_{tag}"] = a, b, O.matmul(a, b)
    x = synth.normal((16, 64), seed=0, tensor_id=0)
    w = synth.uniform((48, 64), -1 / 8, 1 / 8, seed=0, tensor_id=1)
    bias = synth.uniform((48,), -1 / 8, 1 / 8, seed=0, tensor_id=2)
    out["linear_x"], out["linear_w"], out["linear_b"] = x, w, bias
    out["linear_y"] = O.linear_forward(x, w, bias)
    meta = ("Tensor::matmul -> matmul_blocked (ghostflow-core/src/ops/matmul.rs:91-119) on "
            f"A ~ N(0,1) (seed 0, id 0), B ~ N(0,1) (seed 0, id 1), shapes m x k x n {GEMM_SHAPES}; "
            "Linear::forward (ghostflow-nn/src/linear.rs:56-69) x [16,64] ~ N(0,1), W [48,64], "
            "b [48] ~ U(-1/8, 1/8) (ids 1, 2)")
    return out, meta


def quant():
    out = {}
    cases = {
        "ref_per_tensor_sym": (np.arange(1, 7, dtype=np.float32).reshape(2, 3), "tensor", True),
        "ref_per_channel_sym": (np.array([[1, 2, 3], [10, 20, 30]], np.float32), "channel", True),
        "ref_asym": (np.array([-5, -3, -1, 1, 3, 5], np.float32), "tensor", False),
        "ref_activation": (np.array([0.5, 1.5, 2.5], np.float32), "tensor", False),
        "ties": (np.array([2.5, -2.5, 0.5, -0.5, 127.0, 1.5], np.float32), "tensor", True),
    }
    rnd = synth.normal((37, 129), 0.0, 0.02, seed=0, tensor_id=3)
    for sym in (True, False):
        cases[f"rand_channel_{'sym' if sym else 'asym'}"] = (rnd, "channel", sym)
        cases[f"rand_tensor_{'sym' if sym else 'asym'}"] = (rnd, "tensor", sym)
    for name, (x, kind, sym) in cases.items():
        if kind == "channel":
            q, s, z = O.quantize_per_channel(x, sym)
        else:
            q, s, z = O.quantize_per_tensor(x, sym)
            s, z = np.array([s], np.float32), np.array([z], np.int8)
        out[f"{name}_x"], out[f"{name}_q"], out[f"{name}_s"], out[f"{name}_z"] = x, q, s, z
        out[f"{name}_deq"] = O.dequantize(q, s, z)
        out[f"{name}_kind"] = np.array([kind == "channel", sym], np.bool_)
    meta = ("QuantizedTensor quantize_per_tensor_int8 / quantize_per_channel_int8 / dequantize_int8 "
            "(ghostflow-nn/src/quantization.rs:77-204) on the reference unit-test inputs "
            "(quantization.rs:300-428), exact ties, and x [37,129] ~ N(0, 0.02) (seed 0, id 3); "
            "<name>_kind = [per_channel, symmetric]")
    return out, meta


def qlinear():
    out = {}
    n, k = 48, 64
    w = synth.normal((n, k), 0.0, 0.02, seed=0, tensor_id=1)
    qw, sw, _ = O.quantize_per_channel(w, True)
    bias = synth.uniform((n,), -0.1, 0.1, seed=0, tensor_id=2)
    out["qw"], out["sw"], out["bias"] = qw, sw, bias
    for m in (1, 5):
        x = synth.normal((m, k), seed=m, tensor_id=0)
        qx, sx, zx = O.quantize_per_tensor(x, False)
        y, acc = O.qlinear_i8(qx, sx, zx, False, qw, sw, bias)
        out[f"m{m}_qx"], out[f"m{m}_sx"], out[f"m{m}_zx"] = qx, np.array([sx]), np.array([zx])
        out[f"m{m}_y"], out[f"m{m}_acc"] = y, acc
        # per-row symmetric activations (QuantizationConfig::default)
        qr, sr, zr = O.quantize_per_channel(x, True)
        yr, accr = O.qlinear_i8(qr, sr, zr, True, qw, sw, None)
        out[f"m{m}_row_qx"], out[f"m{m}_row_sx"], out[f"m{m}_row_zx"] = qr, sr, zr
        out[f"m{m}_row_y"], out[f"m{m}_row_acc"] = yr, accr
    meta = ("INT8 linear on the reference scheme: W [48,64] ~ N(0,0.02) (seed 0, id 1) per-channel "
            "symmetric; x [m,64] ~ N(0,1) (seed m, id 0), m in {1,5}, per-tensor asymmetric "
            "(DynamicQuantization::quantize_activation, quantization.rs:280-287) with bias "
            "~ U(-0.1,0.1) (id 2), and per-row symmetric without bias")
    return out, meta


def gemv():
    b, k, n = 3, 64, 80
    x = synth.normal((b, k), seed=0, tensor_id=0)
    w = synth.normal((k, n), 0.0, 0.02, seed=0, tensor_id=1)
    qw, s, z = O.quantize_per_channel(w, True)
    qa, sa, za = O.quantize_per_channel(w, False)
    out = {"x": x, "w": w, "y": O.matmul(x, w), "qw": qw, "s": s, "z": z,
           "y_w8": O.matmul(x, O.dequantize(qw, s, z)),
           "qa": qa, "sa": sa, "za": za, "y_w8_asym": O.matmul(x, O.dequantize(qa, sa, za))}
    meta = ("Decode GEMV = Tensor::matmul at M = 3 (matmul.rs:91-119): x [3,64] ~ N(0,1), "
            "W [64,80] ~ N(0,0.02) (seed 0, ids 0, 1); int8 weights quantized per channel over "
            "dim 0 (symmetric and asymmetric), reference composite get_weights -> matmul")
    return out, meta


def sdpa():
    out = {}
    for s in (8, 37):
        q = synth.normal((1, 2, s, 16), seed=0, tensor_id=0)
        k = synth.normal((1, 2, s, 16), seed=0, tensor_id=1)
        v = synth.normal((1, 2, s, 16), seed=0, tensor_id=2)
        out[f"s{s}_q"], out[f"s{s}_k"], out[f"s{s}_v"] = q, k, v
        o, w = O.sdpa(q, k, v, want_weights=True)
        out[f"s{s}_out"], out[f"s{s}_weights"] = o, w
        sc = np.float32(1.0) / np.sqrt(np.float32(16))
        out[f"s{s}_causal_out"] = O.flash_attention(q, k, v, sc, True)
    x = synth.normal((5, 100), 0.0, 3.0, seed=0, tensor_id=4)
    out["softmax_x"], out["softmax_y"] = x, O.softmax_lastdim(x)
    meta = ("scaled_dot_product_attention (ghostflow-nn/src/attention.rs:11-49, no mask) with "
            "weights, and flash_attention causal (ghostflow-cuda/src/ops.rs:166-224), Q/K/V "
            "[1,2,S,16] ~ N(0,1) (seed 0, ids 0-2), S in {8,37}; softmax(-1) "
            "(activation.rs:165-216) of x [5,100] ~ N(0,3) (id 4)")
    return out, meta


GROUPS = {"gemm": gemm, "quant": quant, "qlinear": qlinear, "gemv": gemv, "sdpa": sdpa}


def build(name):
    arrays, meta = GROUPS[name]()
    arrays["meta"] = np.array(meta)
    return arrays


def main():
    for name in GROUPS:
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **build(name))
        print("wrote", os.path.relpath(path, ROOT), os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
