"""ctypes wrapper over oracle/libgf_oracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle is the CPU restatement of GhostFlow's hot path (see gf_oracle.c
for the reference file:line each function follows).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only as the checker / the timed CPU baseline -- never as the product.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libgf_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build() -> None:
    """Compile the oracle with its Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.gfo_matmul_blocked.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz]
        L.gfo_batched_matmul.argtypes = [_f32p, _sz, _f32p, _sz, _f32p, _sz, _sz, _sz, _sz]
        _szp = np.ctypeslib.ndpointer(np.uintp, flags="C_CONTIGUOUS")
        L.gfo_broadcast_binary.argtypes = [C.c_int, _f32p, _szp, _sz, _f32p, _szp, _sz, _f32p, _szp, _sz]
        L.gfo_transpose_last2.argtypes = [_f32p, _f32p, _sz, _sz, _sz]
        L.gfo_matmul_backward.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, C.c_void_p, C.c_void_p]
        L.gfo_add_row_bias.argtypes = [_f32p, _f32p, _sz, _sz]
        L.gfo_mul_scalar.argtypes = [_f32p, _sz, C.c_float]
        L.gfo_linear_forward.argtypes = [_f32p, _f32p, C.c_void_p, _f32p, _sz, _sz, _sz]
        L.gfo_linear_forward.restype = C.c_int
        L.gfo_softmax_lastdim.argtypes = [_f32p, _f32p, _sz, _sz]
        L.gfo_silu_mul.argtypes = [_f32p, _f32p, _f32p, _sz]
        L.gfo_apply_mask_cycled.argtypes = [_f32p, _sz, _f32p, _sz]
        L.gfo_apply_causal.argtypes = [_f32p, _sz, _sz]
        L.gfo_sdpa.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, _sz, _f32p, C.c_void_p,
                               _sz, _sz, _sz, _sz]
        L.gfo_sdpa.restype = C.c_int
        L.gfo_flash_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz,
                                          C.c_float, C.c_int]
        L.gfo_flash_attention.restype = C.c_int
        L.gfo_flash_attention_rows.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz,
                                               C.c_float, C.c_int, _sz, _sz]
        L.gfo_flash_attention_rows.restype = C.c_int
        L.gfo_flash_attention_blockwise.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz,
                                                    _sz, _sz, C.c_int, C.c_float]
        L.gfo_flash_attention_blockwise.restype = C.c_int
        L.gfo_quantize_per_tensor.argtypes = [_f32p, _sz, C.c_int, _i8p,
                                              C.POINTER(C.c_float), C.POINTER(C.c_int8)]
        L.gfo_quantize_per_channel.argtypes = [_f32p, _sz, _sz, C.c_int, _i8p, _f32p, _i8p]
        L.gfo_dequantize.argtypes = [_i8p, _sz, _sz, _f32p, _i8p, _sz, _f32p]
        L.gfo_qlinear_i8.argtypes = [_i8p, _f32p, C.c_void_p, C.c_int, _i8p, _f32p,
                                     C.c_void_p, C.c_void_p, C.c_void_p, _sz, _sz, _sz]
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# -- ghostflow-core ---------------------------------------------------------

def matmul(a, b):
    """Tensor::matmul on 2-D operands (matmul.rs:13-57 -> matmul_blocked)."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"ShapeMismatch expected [{m}, {k}] got [{k2}, {n}]")
    c = np.empty((m, n), np.float32)
    lib().gfo_matmul_blocked(a, b, c, m, k, n)
    return c


def batched_matmul(a, b):
    """matmul.rs:122-170 (batch dims flattened; modulo batch indexing)."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape[-2:]
    n = b.shape[-1]
    ab = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    bb = int(np.prod(b.shape[:-2])) if b.ndim > 2 else 1
    batch_shape = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    batch = int(np.prod(batch_shape)) if batch_shape else 1
    c = np.empty(tuple(batch_shape) + (m, n), np.float32)
    lib().gfo_batched_matmul(a, ab, b, bb, c, batch, m, k, n)
    return c


def broadcast_binary(a, b, op):
    """Tensor::add / Tensor::mul (arithmetic.rs:19-45, broadcast_binary_op
    :123-215); op is "add" or "mul".  Result dims by Shape::broadcast_with
    (shape.rs:49-80); ValueError where the shapes do not broadcast."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nd = max(a.ndim, b.ndim)
    dims = []
    for i in range(nd):
        x = a.shape[a.ndim - 1 - i] if i < a.ndim else 1
        y = b.shape[b.ndim - 1 - i] if i < b.ndim else 1
        if x == y or y == 1:
            dims.append(x)
        elif x == 1:
            dims.append(y)
        else:
            raise ValueError(f"BroadcastError a {list(a.shape)} b {list(b.shape)}")
    dims = dims[::-1]
    c = np.empty(dims, np.float32)
    ad = np.array(a.shape or (1,), np.uintp)
    bd = np.array(b.shape or (1,), np.uintp)
    cd = np.array(dims or [1], np.uintp)
    lib().gfo_broadcast_binary({"add": 0, "mul": 1}[op], np.ascontiguousarray(a).reshape(-1), ad, a.ndim,
                               np.ascontiguousarray(b).reshape(-1), bd, b.ndim, c.reshape(-1), cd, len(dims))
    return c


def transpose_last2(x):
    x = _f32(x)
    r, c = x.shape[-2:]
    batch = int(np.prod(x.shape[:-2])) if x.ndim > 2 else 1
    out = np.empty(x.shape[:-2] + (c, r), np.float32)
    lib().gfo_transpose_last2(x, out, batch, r, c)
    return out


def matmul_backward(grad, a, b):
    """matmul_backward (ghostflow-autograd/src/backward.rs:131-160):
    (grad . b^T, a^T . grad) for grad [m,n], a [m,k], b [k,n]."""
    grad, a, b = _f32(grad), _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    if b.shape[0] != k or grad.shape != (m, n):
        raise ValueError("matmul_backward: shape mismatch")
    ga = np.empty((m, k), np.float32)
    gb = np.empty((k, n), np.float32)
    lib().gfo_matmul_backward(grad, a, b, m, k, n, _ptr(ga), _ptr(gb))
    return ga, gb


def linear_forward(x, w, bias=None):
    """Linear::forward (linear.rs:56-69): x W^T + b."""
    x, w = _f32(x), _f32(w)
    m, in_f = x.shape
    out_f = w.shape[0]
    y = np.empty((m, out_f), np.float32)
    b = None if bias is None else _f32(bias)
    rc = lib().gfo_linear_forward(x, w, _ptr(b), y, m, in_f, out_f)
    if rc:
        raise MemoryError("oracle allocation failed")
    return y


def silu_mul(gate, up):
    """gate.silu().mul(&up) (activation.rs:117-122, arithmetic.rs:39-45)."""
    g, u = _f32(gate), _f32(up)
    if g.shape != u.shape:
        raise ValueError("gate and up must have the same shape")
    out = np.empty(g.shape, np.float32)
    lib().gfo_silu_mul(g.reshape(-1), u.reshape(-1), out.reshape(-1), g.size)
    return out


def swiglu_forward(x, wg, bg, wu, bu, wd, bd):
    """SwiGLU::forward (ghostflow-nn/src/llama.rs:276-286): three
    Linear::forward calls and the silu * up product, composed from the
    restated pieces.  Returns (y, h) with h = silu(gate) * up."""
    gate = linear_forward(x, wg, bg)
    up = linear_forward(x, wu, bu)
    h = silu_mul(gate, up)
    return linear_forward(h, wd, bd), h


def softmax_lastdim(x):
    x = _f32(x)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    y = np.empty_like(x)
    lib().gfo_softmax_lastdim(x, y, rows, cols)
    return y


def sdpa(q, k, v, mask=None, want_weights=False):
    """scaled_dot_product_attention (attention.rs:11-49), q/k/v [..., S, D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    sq, d = q.shape[-2:]
    skv = k.shape[-2]
    bh = q.size // (sq * d) if q.size else 0
    out = np.empty(q.shape, np.float32)
    w = np.empty(q.shape[:-2] + (sq, skv), np.float32) if want_weights else None
    mk = None if mask is None else _f32(mask)
    rc = lib().gfo_sdpa(q, k, v, _ptr(mk), 0 if mk is None else mk.size, out, _ptr(w),
                        bh, sq, skv, d)
    if rc:
        raise MemoryError("oracle allocation failed")
    return (out, w) if want_weights else out


def mha_forward_with_cache(query, key, value, wq, bq, wk, bk, wv, bv, wo, bo, num_heads,
                           mask=None, past_key=None, past_value=None):
    """MultiHeadAttention::forward_with_cache (ghostflow-nn/src/attention.rs:
    100-144) with dropout off (p = 0 or eval mode, :37-43).

    query [B, S, E], key/value [B, Sk, E]; weights [E, E] as [out, in],
    biases [E] or None; past_key/past_value [B, P, E] (the layout
    concat_tensors joins along dim 1, :214-247).  Returns (output [B, S, E],
    attn_weights [B, H, S, P + Sk], k_new, v_new) where k_new/v_new are the
    new projected keys/values only (:141-142), given as [B, Sk, E]: the
    storage order of the reference's [B, H, Sk, D] view (reshape, then
    transpose(1, 2), :146-150).

    All arithmetic is in the C restatement: linear_forward (Linear::forward
    on [B*S, E]; the batched 3-D form of :61 sums each element in the same
    sequential-k order, matmul.rs:147-160) and sdpa (:11-49).  What numpy
    does here is data movement only: the head split/merge of
    reshape_for_attention / reshape_from_attention (:146-157) and the
    concatenation.
    """
    query, key, value = _f32(query), _f32(key), _f32(value)
    b, s, e = query.shape
    sk = key.shape[1]
    h = int(num_heads)
    d = e // h
    q = linear_forward(query.reshape(b * s, e), wq, bq).reshape(b, s, e)
    k = linear_forward(key.reshape(b * sk, e), wk, bk).reshape(b, sk, e)
    v = linear_forward(value.reshape(b * sk, e), wv, bv).reshape(b, sk, e)
    if past_key is not None and past_value is not None:
        kc = np.concatenate([_f32(past_key), k], axis=1)
        vc = np.concatenate([_f32(past_value), v], axis=1)
    else:
        kc, vc = k, v
    skv = kc.shape[1]

    def heads(t, n):  # [B, n, E] -> [B, H, n, D], one head at a time (row copies of D floats)
        src = t.reshape(b, n, h, d)
        out = np.empty((b, h, n, d), np.float32)
        for hh in range(h):
            out[:, hh] = src[:, :, hh, :]
        return out

    out, w = sdpa(heads(q, s), heads(kc, skv), heads(vc, skv), mask=mask, want_weights=True)
    attn = np.ascontiguousarray(out.transpose(0, 2, 1, 3)).reshape(b * s, e)
    output = linear_forward(attn, wo, bo).reshape(b, s, e)
    return output, w, k, v


def flash_attention(q, k, v, scale, causal):
    """ghostflow-cuda ops::attention::flash_attention (ops.rs:166-224)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s, d = q.shape[-2:]
    bh = q.size // (s * d)
    out = np.empty(q.shape, np.float32)
    rc = lib().gfo_flash_attention(q, k, v, out, bh, s, d, float(scale), int(bool(causal)))
    if rc:
        raise MemoryError("oracle allocation failed")
    return out


def flash_attention_rows(q, k, v, scale, causal, r0, r1):
    """Rows [r0, r1) of one (b,h) slice of flash_attention; q/k/v [S, D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s, d = q.shape
    out = np.zeros((s, d), np.float32)
    rc = lib().gfo_flash_attention_rows(q, k, v, out, s, d, float(scale),
                                        int(bool(causal)), r0, r1)
    if rc:
        raise MemoryError("oracle allocation failed")
    return out[r0:r1]


def flash_attention_blockwise(q, k, v, block_m=64, block_n=64, causal=False, scale=1.0):
    """FlashAttention::forward (ghostflow-nn/src/flash_attention.rs:81-250)
    on q [B, Sq, d], k / v [B, Sk, d] with FlashAttentionConfig's block
    sizes, causal flag and scale (the reference's own recurrence, including
    its once-per-key correction)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    bsz, sq, d = q.shape
    sk = k.shape[1]
    out = np.empty((bsz, sq, d), np.float32)
    rc = lib().gfo_flash_attention_blockwise(q.reshape(-1), k.reshape(-1), v.reshape(-1), out.reshape(-1),
                                             bsz, sq, sk, d, int(block_m), int(block_n), int(bool(causal)),
                                             float(scale))
    if rc == 1:
        raise ValueError("block sizes must be positive")
    if rc:
        raise MemoryError("oracle allocation failed")
    return out


# -- ghostflow-nn quantization ----------------------------------------------

def quantize_per_tensor(x, symmetric):
    x = _f32(x)
    q = np.empty(x.shape, np.int8)
    s = C.c_float()
    z = C.c_int8()
    lib().gfo_quantize_per_tensor(x.reshape(-1), x.size, int(bool(symmetric)),
                                  q.reshape(-1), C.byref(s), C.byref(z))
    return q, np.float32(s.value), np.int8(z.value)


def quantize_per_channel(x, symmetric):
    x = _f32(x)
    rows = x.shape[0]
    cols = x.size // rows
    q = np.empty(x.shape, np.int8)
    s = np.empty(rows, np.float32)
    z = np.empty(rows, np.int8)
    lib().gfo_quantize_per_channel(x.reshape(-1), rows, cols, int(bool(symmetric)),
                                   q.reshape(-1), s, z)
    return q, s, z


def dequantize(q, scales, zps):
    q = np.ascontiguousarray(q, np.int8)
    scales = np.ascontiguousarray(np.atleast_1d(scales), np.float32)
    zps = np.ascontiguousarray(np.atleast_1d(zps), np.int8)
    rows = q.shape[0] if q.ndim else 1
    cols = q.size // rows if rows else 0
    out = np.empty(q.shape, np.float32)
    lib().gfo_dequantize(q.reshape(-1), rows, cols, scales, zps, scales.size,
                         out.reshape(-1))
    return out


def qswiglu_forward(x, qwg, swg, bg, qwu, swu, bu, qwd, swd, bd):
    """SwiGLU::forward (llama.rs:276-286) with every Linear run as the INT8
    linear on DynamicQuantization's scheme (quantization.rs:251-288):
    weights per-channel symmetric codes + scales, activations quantized per
    tensor, asymmetric (quantize_activation, :280-287) -- x before gate/up,
    h = silu(gate) * up before down.  Returns a dict of every stage."""
    qx, sx, zx = quantize_per_tensor(x, symmetric=False)
    gate, _ = qlinear_i8(qx, sx, zx, False, qwg, swg, bg, want_acc=False)
    up, _ = qlinear_i8(qx, sx, zx, False, qwu, swu, bu, want_acc=False)
    h = silu_mul(gate, up)
    qh, sh, zh = quantize_per_tensor(h, symmetric=False)
    y, _ = qlinear_i8(qh, sh, zh, False, qwd, swd, bd, want_acc=False)
    return {"qx": qx, "sx": sx, "zx": zx, "gate": gate, "up": up, "h": h, "qh": qh, "sh": sh, "zh": zh,
            "y": y}


def qlinear_i8(qx, sx, zx, x_per_row, qw, sw, bias=None, want_acc=True):
    qx = np.ascontiguousarray(qx, np.int8)
    qw = np.ascontiguousarray(qw, np.int8)
    m, k = qx.shape
    n = qw.shape[0]
    sx = np.ascontiguousarray(np.atleast_1d(sx), np.float32)
    zxa = None if zx is None else np.ascontiguousarray(np.atleast_1d(zx), np.int8)
    sw = np.ascontiguousarray(sw, np.float32)
    b = None if bias is None else _f32(bias)
    y = np.empty((m, n), np.float32)
    acc = np.empty((m, n), np.int32) if want_acc else None
    lib().gfo_qlinear_i8(qx, sx, _ptr(zxa), int(bool(x_per_row)), qw, sw, _ptr(b),
                         _ptr(y), _ptr(acc), m, n, k)
    return y, acc
