"""Thin wrappers that call the C ABI on torch device tensors.

torch only supplies device memory and the current HIP stream; every
computation below is one call into libghostflow_hip.so.  Each wrapper checks
dtype / contiguity / device on the host and raises GhostFlowError with the
library's status code and thread-local message when a call fails.
"""
from __future__ import annotations

import torch

from . import _lib


class GhostFlowError(RuntimeError):
    """A non-zero status from the C ABI (GhostFlowError codes)."""

    def __init__(self, status: int, message: str):
        self.status = status
        name = _lib.STATUS_NAMES.get(status, str(status))
        super().__init__(f"{name}: {message}")


def _check(rc: int) -> None:
    if rc != _lib.SUCCESS:
        msg = _lib.load().gfh_last_error()
        raise GhostFlowError(rc, msg.decode() if msg else "")


def _stream(dev=None) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _workspace_bytes(ws):
    """Bytes a caller workspace holds, whatever its dtype: numel times the
    element size.  The workspace must be a contiguous device tensor."""
    if ws is None:
        return 0
    if not ws.is_cuda:
        raise GhostFlowError(_lib.INVALID_DATA, "workspace must be a device tensor")
    if not ws.is_contiguous():
        raise GhostFlowError(_lib.INVALID_DATA, "workspace must be contiguous")
    return ws.numel() * ws.element_size()


def _workspace(ws):
    """(pointer, bytes) of a caller workspace, (None, 0) without one."""
    return (None, 0) if ws is None else (ws.data_ptr(), _workspace_bytes(ws))


def _need(t, dtype, name):
    if t is None:
        return
    if not t.is_cuda:
        raise GhostFlowError(_lib.INVALID_DATA, f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise GhostFlowError(_lib.INVALID_DATA, f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise GhostFlowError(_lib.INVALID_DATA, f"{name} must be contiguous")


def lib():
    return _lib.load()


def init() -> None:
    _check(lib().gfh_init())


def set_pointer_checks(enabled: bool) -> None:
    _check(lib().gfh_set_pointer_checks(1 if enabled else 0))


# ---- fp32 GEMM --------------------------------------------------------------

def sgemm(a, b, *, trans_a=False, trans_b=False, alpha=1.0, beta=0.0, bias=None, out=None):
    """out = alpha * op(a) @ op(b) + beta * out (+ bias), 2-D row-major."""
    _need(a, torch.float32, "a")
    _need(b, torch.float32, "b")
    _need(bias, torch.float32, "bias")
    m, k = (a.shape[1], a.shape[0]) if trans_a else (a.shape[0], a.shape[1])
    k2, n = (b.shape[1], b.shape[0]) if trans_b else (b.shape[0], b.shape[1])
    if k != k2:
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch expected [{m}, {k}] got [{k2}, {n}]")
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    _need(out, torch.float32, "out")
    _check(lib().gfh_sgemm(int(trans_a), int(trans_b), m, n, k, float(alpha), a.data_ptr(),
                           max(a.shape[1], 1), b.data_ptr(), max(b.shape[1], 1),
                           float(beta), out.data_ptr(), max(n, 1), _ptr(bias), _stream(a.device)))
    return out


def matmul(a, b):
    """Tensor::matmul (ghostflow-core/src/ops/matmul.rs:13-42): 2-D -> GEMM,
    otherwise the batched form with modulo batch indexing (:122-170)."""
    _need(a, torch.float32, "a")
    _need(b, torch.float32, "b")
    if a.dim() < 2 or b.dim() < 2:
        raise GhostFlowError(_lib.INVALID_SHAPE, "matmul requires at least 2D tensors")
    m, k = a.shape[-2:]
    k2, n = b.shape[-2:]
    if k != k2:
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch expected [{m}, {k}] got [{k2}, {n}]")
    if a.dim() == 2 and b.dim() == 2:
        return sgemm(a, b)
    batch_shape = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    batch = 1
    for s in batch_shape:
        batch *= s
    ba = 1
    for s in a.shape[:-2]:
        ba *= s
    bb = 1
    for s in b.shape[:-2]:
        bb *= s
    out = torch.empty(tuple(batch_shape) + (m, n), dtype=torch.float32, device=a.device)
    _check(lib().gfh_sgemm_strided_batched(0, 0, m, n, k, 1.0, a.data_ptr(), k, m * k, max(ba, 1),
                                           b.data_ptr(), n, k * n, max(bb, 1), 0.0, out.data_ptr(),
                                           n, m * n, batch, None, _stream(a.device)))
    return out


def linear(x, weight, bias=None):
    """Linear::forward (ghostflow-nn/src/linear.rs:56-69): x @ W^T + b."""
    return sgemm(x, weight, trans_b=True, bias=bias)


# ---- int8 quantization ---------------------------------------------------------

def matmul_backward(grad, a, b, *, need_a=True, need_b=True):
    """matmul_backward (ghostflow-autograd/src/backward.rs:131-160) for
    C = a @ b: returns (grad @ b^T, a^T @ grad); a part not needed is None."""
    for t, n in ((grad, "grad"), (a, "a"), (b, "b")):
        _need(t, torch.float32, n)
    m, k = a.shape
    n = b.shape[1]
    if b.shape[0] != k or tuple(grad.shape) != (m, n):
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch a {list(a.shape)} b {list(b.shape)} "
                             f"grad {list(grad.shape)}")
    ga = torch.empty((m, k), dtype=torch.float32, device=a.device) if need_a else None
    gb = torch.empty((k, n), dtype=torch.float32, device=a.device) if need_b else None
    _check(lib().gfh_matmul_backward_f32(grad.data_ptr(), a.data_ptr(), b.data_ptr(), m, k, n, _ptr(ga), _ptr(gb),
                                         _stream(a.device)))
    return ga, gb


def quantize_per_channel(x, symmetric=True):
    _need(x, torch.float32, "x")
    rows = x.shape[0]
    cols = x.numel() // rows if rows else 0
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
    z = torch.empty(rows, dtype=torch.int8, device=x.device)
    _check(lib().gfh_quantize_i8_per_channel(x.data_ptr(), rows, cols, int(bool(symmetric)),
                                             q.data_ptr(), s.data_ptr(), z.data_ptr(),
                                             _stream(x.device)))
    return q, s, z


def quantize_per_tensor(x, symmetric=False, workspace=None):
    _need(x, torch.float32, "x")
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(1, dtype=torch.float32, device=x.device)
    z = torch.empty(1, dtype=torch.int8, device=x.device)
    ws_ptr, ws_bytes = _workspace(workspace)
    _check(lib().gfh_quantize_i8_per_tensor(x.data_ptr(), x.numel(), int(bool(symmetric)),
                                            q.data_ptr(), s.data_ptr(), z.data_ptr(),
                                            ws_ptr, ws_bytes, _stream(x.device)))
    return q, s, z


def quantize_per_tensor_workspace_size(n: int) -> int:
    return int(lib().gfh_quantize_i8_per_tensor_workspace_size(n))


def dequantize(q, scales, zero_points):
    _need(q, torch.int8, "q")
    _need(scales, torch.float32, "scales")
    _need(zero_points, torch.int8, "zero_points")
    rows = q.shape[0] if q.dim() else 1
    cols = q.numel() // rows if rows else 0
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    _check(lib().gfh_dequantize_i8(q.data_ptr(), rows, cols, scales.data_ptr(), zero_points.data_ptr(),
                                   scales.numel(), out.data_ptr(), _stream(q.device)))
    return out


def qweight_rowsum(qw):
    _need(qw, torch.int8, "qw")
    n, k = qw.shape
    out = torch.empty(n, dtype=torch.int32, device=qw.device)
    _check(lib().gfh_qweight_rowsum(qw.data_ptr(), n, k, out.data_ptr(), _stream(qw.device)))
    return out


def qlinear(qx, sx, zx, qw, sw, *, x_per_row=False, w_rowsum=None, bias=None, want_y=True,
            want_acc=False):
    _need(qx, torch.int8, "qx")
    _need(qw, torch.int8, "qw")
    _need(sx, torch.float32, "sx")
    _need(sw, torch.float32, "sw")
    _need(zx, torch.int8, "zx")
    _need(w_rowsum, torch.int32, "w_rowsum")
    _need(bias, torch.float32, "bias")
    m, k = qx.shape
    n = qw.shape[0]
    if qw.shape[1] != k:
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch expected [{m}, {k}] got [{qw.shape[1]}, {n}]")
    if zx is not None and w_rowsum is None:
        w_rowsum = qweight_rowsum(qw)
    y = torch.empty((m, n), dtype=torch.float32, device=qx.device) if want_y else None
    acc = torch.empty((m, n), dtype=torch.int32, device=qx.device) if want_acc else None
    _check(lib().gfh_qlinear_i8(qx.data_ptr(), _ptr(sx), _ptr(zx), int(bool(x_per_row)), qw.data_ptr(),
                                _ptr(sw), _ptr(w_rowsum), _ptr(bias), _ptr(y), _ptr(acc), m, n, k,
                                _stream(qx.device)))
    return y, acc


def qlinear_dynamic(x, qw, sw, w_rowsum, *, bias=None, out=None, workspace=None):
    """The INT8 linear on fp32 activations x [m, k]: quantize_activation
    (per tensor, asymmetric, quantization.rs:280-287) then qlinear with the
    per-channel weight codes qw [n, k]; y [m, n].  Same codes and outputs as
    quantize_per_tensor followed by qlinear, in one launch for m <= 4."""
    _need(x, torch.float32, "x")
    _need(qw, torch.int8, "qw")
    _need(sw, torch.float32, "sw")
    _need(w_rowsum, torch.int32, "w_rowsum")
    _need(bias, torch.float32, "bias")
    m, k = x.shape
    n = qw.shape[0]
    if qw.shape[1] != k:
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch expected [{m}, {k}] got [{qw.shape[1]}, {n}]")
    y = torch.empty((m, n), dtype=torch.float32, device=x.device) if out is None else out
    ws_ptr, ws_bytes = _workspace(workspace)
    _check(lib().gfh_qlinear_dynamic_i8(x.data_ptr(), qw.data_ptr(), sw.data_ptr(), w_rowsum.data_ptr(),
                                        _ptr(bias), y.data_ptr(), m, n, k, ws_ptr, ws_bytes, _stream(x.device)))
    return y


# ---- GEMV ---------------------------------------------------------------------

def gemv_f32(x, w, out=None):
    _need(x, torch.float32, "x")
    _need(w, torch.float32, "w")
    b, k = x.shape
    n = w.shape[1]
    if w.shape[0] != k:
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch expected [{b}, {k}] got [{w.shape[0]}, {n}]")
    y = torch.empty((b, n), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().gfh_gemv_f32(x.data_ptr(), w.data_ptr(), y.data_ptr(), b, k, n, _stream(x.device)))
    return y


def gemv_w8(x, qw, scales, zero_points=None, out=None):
    _need(x, torch.float32, "x")
    _need(qw, torch.int8, "qw")
    _need(scales, torch.float32, "scales")
    _need(zero_points, torch.int8, "zero_points")
    b, k = x.shape
    n = qw.shape[1]
    if qw.shape[0] != k:
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch expected [{b}, {k}] got [{qw.shape[0]}, {n}]")
    y = torch.empty((b, n), dtype=torch.float32, device=x.device) if out is None else out
    _check(lib().gfh_gemv_w8(x.data_ptr(), qw.data_ptr(), scales.data_ptr(), _ptr(zero_points),
                             y.data_ptr(), b, k, n, _stream(x.device)))
    return y


# ---- attention ------------------------------------------------------------------

def softmax_lastdim(x, out=None):
    _need(x, torch.float32, "x")
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    y = torch.empty_like(x) if out is None else out
    _check(lib().gfh_softmax_lastdim_f32(x.data_ptr(), y.data_ptr(), rows, cols, _stream(x.device)))
    return y


def sdpa(q, k, v, *, scale=None, causal=False, mask=None, want_weights=False, out=None):
    """Fused scaled_dot_product_attention on [B, H, S, D] tensors."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, torch.float32, nm)
    _need(mask, torch.float32, "mask")
    b, h, sq, d = q.shape
    skv = k.shape[2]
    if scale is None:
        scale = _inv_sqrt(d)
    o = torch.empty_like(q) if out is None else out
    w = torch.empty((b, h, sq, skv), dtype=torch.float32, device=q.device) if want_weights else None
    _check(lib().gfh_sdpa_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), _ptr(w), b, h, sq,
                              skv, d, float(scale), int(bool(causal)), _ptr(mask),
                              0 if mask is None else mask.numel(), _stream(q.device)))
    return (o, w) if want_weights else o


def flash_attention_blockwise(q, k, v, *, block_size_m=64, block_size_n=64, causal=False, scale=1.0,
                              out=None, workspace=None):
    """FlashAttention::forward (ghostflow-nn/src/flash_attention.rs:81-250)
    on q [B, Sq, d], k / v [B, Sk, d]: the reference's blockwise recurrence
    with its block sizes, causal flag (top-left j > i) and scale, including
    its once-per-key correction (softmax attention only at block_size_n ==
    1).  Errors as the reference: non-3-D inputs, a d_model mismatch."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, torch.float32, nm)
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise GhostFlowError(_lib.INVALID_SHAPE, "Expected 3D tensors [batch, seq_len, d_model]")
    b, sq, d = q.shape
    sk = k.shape[1]
    if k.shape[2] != d or v.shape[2] != d:
        raise GhostFlowError(_lib.INVALID_SHAPE, "Key and Value must have same d_model as Query")
    if k.shape[0] != b or v.shape[0] != b or v.shape[1] != sk:
        raise GhostFlowError(_lib.INVALID_SHAPE, "key / value must be [batch, seq_len_k, d_model] like query")
    o = torch.empty_like(q) if out is None else out
    _check(lib().gfh_flash_attention_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, sq, sk, d,
                                         int(block_size_m), int(block_size_n), int(bool(causal)), float(scale),
                                         _ptr(workspace), _workspace_bytes(workspace), _stream(q.device)))
    return o


def kv_attention(q, k_cache, v_cache, kv_len, num_heads, *, scale=None, causal=False, mask=None,
                 want_weights=False, out=None):
    """Attention of q [B, Sq, E] over the first kv_len rows of the caches
    [B, C, E] (head h = columns h*D .. h*D+D-1, D = E / num_heads): the
    scaled_dot_product_attention step of MultiHeadAttention::
    forward_with_cache (ghostflow-nn/src/attention.rs:100-144) with the
    concatenated keys read in place.  Returns out [B, Sq, E] (and the
    [B, H, Sq, kv_len] weights)."""
    for t, nm in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _need(t, torch.float32, nm)
    _need(mask, torch.float32, "mask")
    b, sq, e = q.shape
    cap = k_cache.shape[1]
    if tuple(k_cache.shape) != (b, cap, e) or tuple(v_cache.shape) != (b, cap, e):
        raise GhostFlowError(_lib.INVALID_SHAPE, "k_cache / v_cache must be [B, C, E] like q")
    if e % num_heads:
        raise GhostFlowError(_lib.INVALID_SHAPE, "embed_dim must be divisible by num_heads")
    d = e // num_heads
    if scale is None:
        scale = _inv_sqrt(d)
    o = torch.empty_like(q) if out is None else out
    w = torch.empty((b, num_heads, sq, kv_len), dtype=torch.float32, device=q.device) if want_weights else None
    _check(lib().gfh_kv_attention_f32(q.data_ptr(), e, k_cache.data_ptr(), v_cache.data_ptr(), cap, e,
                                      o.data_ptr(), e, _ptr(w), b, num_heads, sq, kv_len, d, float(scale),
                                      int(bool(causal)), _ptr(mask), 0 if mask is None else mask.numel(),
                                      _stream(q.device)))
    return (o, w) if want_weights else o


def _inv_sqrt(d):
    """1.0f32 / (d as f32).sqrt() (attention.rs:19-20), in float32."""
    return float(torch.tensor(1.0, dtype=torch.float32) / torch.sqrt(torch.tensor(float(d), dtype=torch.float32)))


# ---- multi-head attention with a key/value cache ------------------------------------

def mha_workspace_size(b: int, sq: int, e: int) -> int:
    return int(lib().gfh_mha_workspace_size(b, sq, e))


def mha_forward_cached(query, key, value, wq, bq, wk, bk, wv, bv, wo, bo, num_heads, k_cache, v_cache,
                       past_len, *, mask=None, causal=False, want_weights=False, out=None, workspace=None):
    """MultiHeadAttention::forward_with_cache on an in-place cache: writes
    the projected key/value rows into k_cache / v_cache [B, C, E] at
    [past_len, past_len + Sk) and attends over rows [0, past_len + Sk).
    Returns out [B, Sq, E] (and the [B, H, Sq, past_len + Sk] weights)."""
    for t, nm in ((query, "query"), (key, "key"), (value, "value"), (wq, "wq"), (wk, "wk"), (wv, "wv"),
                  (wo, "wo"), (bq, "bq"), (bk, "bk"), (bv, "bv"), (bo, "bo"), (k_cache, "k_cache"),
                  (v_cache, "v_cache"), (mask, "mask")):
        _need(t, torch.float32, nm)
    b, sq, e = query.shape
    sk = key.shape[1]
    if tuple(key.shape) != (b, sk, e) or tuple(value.shape) != (b, sk, e):
        raise GhostFlowError(_lib.INVALID_SHAPE, "key / value must be [B, Sk, E] like query")
    cap = k_cache.shape[1]
    if tuple(k_cache.shape) != (b, cap, e) or tuple(v_cache.shape) != (b, cap, e):
        raise GhostFlowError(_lib.INVALID_SHAPE, "k_cache / v_cache must be [B, C, E]")
    kv_len = past_len + sk
    o = torch.empty_like(query) if out is None else out
    w = (torch.empty((b, num_heads, sq, kv_len), dtype=torch.float32, device=query.device)
         if want_weights else None)
    ws_ptr, ws_bytes = _workspace(workspace)
    _check(lib().gfh_mha_forward_with_cache_f32(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), wq.data_ptr(), _ptr(bq), wk.data_ptr(), _ptr(bk),
        wv.data_ptr(), _ptr(bv), wo.data_ptr(), _ptr(bo), k_cache.data_ptr(), v_cache.data_ptr(), cap, past_len,
        _ptr(mask), 0 if mask is None else mask.numel(), int(bool(causal)), o.data_ptr(), _ptr(w), b, sq, sk, e,
        num_heads, ws_ptr, ws_bytes, _stream(query.device)))
    return (o, w) if want_weights else o


def mha_forward_with_cache(query, key, value, wq, bq, wk, bk, wv, bv, wo, bo, num_heads, mask=None,
                           past_key=None, past_value=None):
    """The reference's signature and results (attention.rs:100-144):
    past_key / past_value [B, P, E] are concatenated before the new keys
    along dim 1; returns (output [B, Sq, E], attn_weights
    [B, H, Sq, P + Sk], k_cache, v_cache), the last two being the new
    projected keys / values as [B, H, Sk, D] views, like
    reshape_for_attention's (:146-150)."""
    b, sq, e = query.shape
    sk = key.shape[1]
    have_past = past_key is not None and past_value is not None
    p = past_key.shape[1] if have_past else 0
    kc = torch.empty((b, p + sk, e), dtype=torch.float32, device=query.device)
    vc = torch.empty_like(kc)
    if p:
        kc[:, :p].copy_(past_key)
        vc[:, :p].copy_(past_value)
    out, w = mha_forward_cached(query, key, value, wq, bq, wk, bk, wv, bv, wo, bo, num_heads, kc, vc, p,
                                mask=mask, want_weights=True)
    d = e // num_heads
    k_new = kc[:, p:].reshape(b, sk, num_heads, d).transpose(1, 2)
    v_new = vc[:, p:].reshape(b, sk, num_heads, d).transpose(1, 2)
    return out, w, k_new, v_new


# ---- SwiGLU feed-forward block (ghostflow-nn/src/llama.rs:259-287) -------------

def silu_mul(gate, up, out=None):
    """gate.silu().mul(&up): silu(v) = v / (1 + exp(-v)) (activation.rs:117-122)."""
    _need(gate, torch.float32, "gate")
    _need(up, torch.float32, "up")
    if gate.shape != up.shape:
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch {list(gate.shape)} vs {list(up.shape)}")
    if out is None:
        out = torch.empty_like(gate)
    _need(out, torch.float32, "out")
    _check(lib().gfh_silu_mul_f32(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
                                  _stream(gate.device)))
    return out


def _swiglu_dims(x, w_gate, w_down):
    if x.dim() != 2:
        raise GhostFlowError(_lib.INVALID_SHAPE, "x must be [m, hidden]")
    m, hidden = x.shape
    inter = w_gate.shape[0]
    if w_gate.shape[1] != hidden or tuple(w_down.shape) != (hidden, inter):
        raise GhostFlowError(_lib.INVALID_SHAPE, f"ShapeMismatch x [{m}, {hidden}] with gate "
                             f"{list(w_gate.shape)} and down {list(w_down.shape)}")
    return m, hidden, inter


def swiglu(x, wg, bg, wu, bu, wd, bd, *, want_h=False):
    """SwiGLU::forward (llama.rs:276-286) in fp32; returns y, or (y, h) with
    h = silu(gate) * up when want_h."""
    for t, n in ((x, "x"), (wg, "wg"), (bg, "bg"), (wu, "wu"), (bu, "bu"), (wd, "wd"), (bd, "bd")):
        _need(t, torch.float32, n)
    m, hidden, inter = _swiglu_dims(x, wg, wd)
    y = torch.empty((m, hidden), dtype=torch.float32, device=x.device)
    h = torch.empty((m, inter), dtype=torch.float32, device=x.device) if want_h else None
    _check(lib().gfh_swiglu_f32(x.data_ptr(), m, hidden, inter, wg.data_ptr(), _ptr(bg), wu.data_ptr(),
                                _ptr(bu), wd.data_ptr(), _ptr(bd), y.data_ptr(), _ptr(h), None, 0,
                                _stream(x.device)))
    return (y, h) if want_h else y


def qswiglu(x, gate, up, down, *, want_h=False):
    """SwiGLU::forward with each Linear as the INT8 linear on
    DynamicQuantization's scheme (quantization.rs:251-288).  gate / up / down
    are (codes, scales, rowsums, bias-or-None) of per-channel symmetric
    weights [out, in]; x and h are quantized per tensor (asymmetric) on the
    device."""
    _need(x, torch.float32, "x")
    for name, (q, s, r, b) in (("gate", gate), ("up", up), ("down", down)):
        _need(q, torch.int8, name + " codes")
        _need(s, torch.float32, name + " scales")
        _need(r, torch.int32, name + " rowsums")
        _need(b, torch.float32, name + " bias")
    m, hidden, inter = _swiglu_dims(x, gate[0], down[0])
    y = torch.empty((m, hidden), dtype=torch.float32, device=x.device)
    h = torch.empty((m, inter), dtype=torch.float32, device=x.device) if want_h else None
    args = []
    for q, s, r, b in (gate, up, down):
        args += [q.data_ptr(), s.data_ptr(), r.data_ptr(), _ptr(b)]
    _check(lib().gfh_swiglu_i8(x.data_ptr(), m, hidden, inter, *args, y.data_ptr(), _ptr(h), None, 0,
                               _stream(x.device)))
    return (y, h) if want_h else y


# ---- state dict files (ghostflow-core/src/serialize.rs) -------------------------

class StateDict:
    """An opened GHOSTFLW / GHOSTFLQ file (gfh_state_dict_open): names,
    shapes and kinds from the mapped header; tensors copied to the device on
    request.  Use as a context manager or call close()."""

    def __init__(self, path: str):
        import ctypes as C
        h = C.c_void_p()
        _check(lib().gfh_state_dict_open(str(path).encode(), C.byref(h)))
        self._h = h
        self._keys = []
        self._info = {}
        for i in range(int(lib().gfh_state_dict_count(h))):
            name, kind, dtype, ndim, nsc = C.c_char_p(), C.c_int(), C.c_int(), C.c_int(), C.c_int64()
            _check(lib().gfh_state_dict_entry(h, i, C.byref(name), C.byref(kind), C.byref(dtype), C.byref(ndim),
                                              None, 0, C.byref(nsc)))
            dims = (C.c_int64 * max(ndim.value, 1))()
            _check(lib().gfh_state_dict_entry(h, i, None, None, None, None, dims, ndim.value, None))
            key = name.value.decode("utf-8")
            self._keys.append(key)
            self._info[key] = (i, kind.value, dtype.value, tuple(dims[d] for d in range(ndim.value)), nsc.value)

    def close(self):
        if self._h:
            lib().gfh_state_dict_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def keys(self):
        return list(self._keys)

    def __contains__(self, key):
        return key in self._info

    def info(self, key):
        """(kind, dtype byte or scheme, shape, nscales)."""
        return self._info[key][1:]

    def tensor(self, key, device="cuda"):
        """A kind-0 entry as a float32 device tensor of its stored shape, or a
        kind-1 entry as (codes int8, scales f32, zero points int8)."""
        idx, kind, _dtype, shape, nsc = self._info[key]
        if kind == 0:
            out = torch.empty(shape, dtype=torch.float32, device=device)
            _check(lib().gfh_state_dict_read_f32(self._h, idx, out.data_ptr(), _stream(out.device)))
            return out
        codes = torch.empty(shape, dtype=torch.int8, device=device)
        scales = torch.empty(nsc, dtype=torch.float32, device=device)
        zps = torch.empty(nsc, dtype=torch.int8, device=device)
        _check(lib().gfh_state_dict_read_q8(self._h, idx, codes.data_ptr(), scales.data_ptr(), zps.data_ptr(),
                                            _stream(codes.device)))
        return codes, scales, zps


def load_state_dict(path, device="cuda"):
    """load_state_dict (serialize.rs:48-88) straight into device memory:
    name -> float32 tensor (GHOSTFLW), or name -> (codes, scales, zero
    points) for the quantized entries of a GHOSTFLQ file."""
    with StateDict(path) as sd:
        return {k: sd.tensor(k, device) for k in sd.keys()}


def save_state_dict(path, state, *, quantized_format=False, dtypes=None):
    """save_state_dict (serialize.rs:20-45) from device tensors, in the
    dict's order.  Values are float32 device tensors, or -- in a GHOSTFLQ
    file -- (codes, scales, zero points) tuples of a QuantizedTensor.
    dtypes optionally maps a name to the dtype byte (or scheme) recorded."""
    import ctypes as C
    entries = (_lib.TensorEntry * max(len(state), 1))()
    keep = []
    dev = None
    for i, (name, v) in enumerate(state.items()):
        e = entries[i]
        nb = str(name).encode("utf-8")
        keep.append(nb)
        e.name = nb
        quant = isinstance(v, (tuple, list))
        t = v[0] if quant else v
        if quant and not quantized_format:
            raise GhostFlowError(_lib.INVALID_DATA, f"{name}: quantized entries need quantized_format=True")
        _need(t, torch.int8 if quant else torch.float32, str(name))
        dev = t.device
        dims = (C.c_int64 * max(t.dim(), 1))(*t.shape)
        keep.append(dims)
        e.kind = 1 if quant else 0
        e.dtype = (dtypes or {}).get(name, 0 if quant else 2)
        e.ndim = t.dim()
        e.dims = C.cast(dims, C.POINTER(C.c_int64))
        e.data = t.data_ptr()
        if quant:
            _need(v[1], torch.float32, f"{name} scales")
            _need(v[2], torch.int8, f"{name} zero points")
            e.scales = v[1].data_ptr()
            e.zero_points = v[2].data_ptr()
            e.nscales = v[1].numel()
    _check(lib().gfh_state_dict_save(str(path).encode(), int(bool(quantized_format)), C.addressof(entries),
                                     len(state), _stream(dev) if dev is not None else None))
