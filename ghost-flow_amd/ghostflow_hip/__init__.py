"""ghostflow_hip -- Python bindings of the gfx950 backend for GhostFlow's dense
hot path (fp32 GEMM / Linear, int8 quantized linear, decode GEMV, SDPA) and
the layers built on it (MultiHeadAttention with a KV cache, SwiGLU).

All compute goes through the C ABI of libghostflow_hip.so
(include/ghostflow_hip.h); see ops.py.  The package lives in the
`ghost-flow_amd/` directory; put that directory on sys.path to import it.
"""
from . import _lib  # noqa: F401
from .ops import (  # noqa: F401
    GhostFlowError,
    StateDict,
    dequantize,
    flash_attention_blockwise,
    gemv_f32,
    gemv_w8,
    init,
    kv_attention,
    lib,
    linear,
    load_state_dict,
    matmul,
    matmul_backward,
    mha_forward_cached,
    mha_forward_with_cache,
    mha_workspace_size,
    qlinear,
    qlinear_dynamic,
    qswiglu,
    quantize_per_channel,
    quantize_per_tensor,
    quantize_per_tensor_workspace_size,
    qweight_rowsum,
    save_state_dict,
    sdpa,
    set_pointer_checks,
    silu_mul,
    sgemm,
    softmax_lastdim,
    swiglu,
)
from .nn import (  # noqa: F401
    FlashAttention,
    FlashAttentionConfig,
    KVCache,
    MultiHeadAttention,
    QuantizedSwiGLU,
    SwiGLU,
)
from .quantization import (  # noqa: F401
    DynamicQuantization,
    QuantizationAwareTraining,
    QuantizationConfig,
    QuantizationScheme,
    QuantizedTensor,
)
from .synth import normal, uniform  # noqa: F401
