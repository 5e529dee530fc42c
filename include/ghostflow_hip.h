/*
 * ghostflow_hip.h -- C ABI of the MI355X (gfx950) backend for GhostFlow's
 * dense hot path.
 *
 * This library takes the role of the reference's `ghostflow-cuda` crate
 * (the L0 device backend): stream-ordered entry points over caller-owned
 * device buffers, plain pointers and sizes, no C++ or HIP types in the
 * signatures.  Citations are file:line in the reference checkout
 * (choksi2212/ghost-flow).
 *
 * Conventions
 *  - Status codes mirror `GhostFlowError` (ghostflow-ffi/src/lib.rs:27-35,
 *    ghostflow-ffi/ghostflow.h:12-20).  On failure `gfh_last_error()` returns
 *    a thread-local message (the reference's ghostflow_get_last_error always
 *    returns "No error", ghostflow-ffi/src/lib.rs:334-337).
 *  - All matrices are row-major and contiguous along their last dimension,
 *    f32 / int8 / int32, as the reference's Tensor storage
 *    (ghostflow-core/src/tensor.rs:19-32).
 *  - Every pointer argument except `stream` and those marked nullable is a
 *    device pointer (hipMalloc / pool memory).  The caller owns all buffers;
 *    the library never frees caller memory (ghostflow-cuda/src/tensor.rs:27-45
 *    holds raw device pointers the same way).
 *  - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *    Calls are asynchronous and ordered on that stream, like the reference's
 *    launchers taking a cudaStream_t (ghostflow-cuda/src/ffi.rs:167-197);
 *    the caller synchronizes.  Shapes, strides and pointers are validated on
 *    the host before any launch; nothing is launched when a call fails.
 *  - Entry points are re-entrant.  Calls that take `workspace` use only that
 *    memory as scratch; when `workspace` is NULL they allocate stream-ordered
 *    scratch (hipMallocAsync/hipFreeAsync) on `stream`.  The *_workspace_size
 *    queries return 0 for shapes their entry point rejects as out of range.
 *  - HIP graphs: calls may be captured on a stream once the same call (same
 *    or larger sizes) has run on that stream outside a capture, with caller
 *    workspaces where a call takes one.  The library's per-stream split-K
 *    buffers are allocated, and their counters zeroed by a kernel, on a
 *    stream's first use; captured calls then allocate nothing and record no
 *    memset.  A call that would allocate on a stream being captured fails
 *    with GFH_ALLOCATION_FAILED before issuing any work.
 */
#ifndef GHOSTFLOW_HIP_H
#define GHOSTFLOW_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GFH_API __attribute__((visibility("default")))

typedef enum gfh_status {
    GFH_SUCCESS = 0,
    GFH_INVALID_SHAPE = 1,
    GFH_INVALID_DATA = 2,
    GFH_NULL_POINTER = 3,
    GFH_ALLOCATION_FAILED = 4,
    GFH_COMPUTATION_FAILED = 5,
    GFH_UNKNOWN = 99
} gfh_status;

typedef void *gfh_stream_t;

/* ---- library ----------------------------------------------------------- */

/* Replaces ghostflow_init (ghostflow-ffi/src/lib.rs:60-64): checks that a
 * gfx950 device is present and caches its properties.  Optional; every entry
 * point initializes lazily. */
GFH_API int gfh_init(void);
/* Releases cached per-device state.  Caller buffers are untouched. */
GFH_API int gfh_shutdown(void);
/* Replaces ghostflow_get_last_error (ghostflow-ffi/src/lib.rs:332-337);
 * thread-local, valid until the next failing call on this thread. */
GFH_API const char *gfh_last_error(void);
/* Replaces ghostflow_version (ghostflow-ffi/src/lib.rs:66-71); static. */
GFH_API const char *gfh_version(void);
/* 1: check that every data pointer is device memory before launching
 * (hipPointerGetAttributes; default), 0: trust the caller. */
GFH_API int gfh_set_pointer_checks(int enabled);

/* ---- fp32 GEMM (Tensor::matmul, Linear) --------------------------------- */

/* C[m,n] = alpha * op(A)[m,k] . op(B)[k,n] + beta * C[m,n] (+ bias[n])
 *   op(A) = A            (trans_a = 0, A is [m, lda >= k])
 *         = A^T          (trans_a = 1, A is [k, lda >= m])
 *   op(B) = B            (trans_b = 0, B is [k, ldb >= n])
 *         = B^T          (trans_b = 1, B is [n, ldb >= k])
 * beta == 0 never reads C.  bias is nullable.  Row-major form of
 * CuBlas::sgemm (ghostflow-cuda/src/blas.rs:70-133; CuBlas::matmul swaps
 * operands to get row-major, :278-313) and of the reference's optional cblas
 * branch (ghostflow-core/src/ops/matmul.rs:60-88).  Serves
 *   Tensor::matmul 2-D   (matmul.rs:13-57, matmul_blocked :91-119): NN
 *   Linear::forward      (ghostflow-nn/src/linear.rs:56-69): x . W^T + b, NT
 *   launch_optimized_sgemm (ghostflow-cuda/src/ffi.rs:169-174). */
GFH_API int gfh_sgemm(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
                      float alpha, const float *a, int64_t lda,
                      const float *b, int64_t ldb, float beta, float *c,
                      int64_t ldc, const float *bias, gfh_stream_t stream);

/* Batched form with the reference's batch indexing: output batch i uses A
 * slice (i % batch_a) and B slice (i % batch_b) (matmul.rs:122-170, :148-149),
 * slices `stride_*` elements apart.  Replaces cublasSgemmBatched
 * (ghostflow-cuda/src/ffi.rs:226-242). */
GFH_API int gfh_sgemm_strided_batched(int trans_a, int trans_b, int64_t m,
                                      int64_t n, int64_t k, float alpha,
                                      const float *a, int64_t lda, int64_t stride_a,
                                      int64_t batch_a, const float *b, int64_t ldb,
                                      int64_t stride_b, int64_t batch_b, float beta,
                                      float *c, int64_t ldc, int64_t stride_c,
                                      int64_t batch, const float *bias,
                                      gfh_stream_t stream);

/* ---- matmul gradient ----------------------------------------------------- */

/* matmul_backward (ghostflow-autograd/src/backward.rs:131-160) for
 * C = A . B with grad = dL/dC [m, n], a [m, k], b [k, n], all row-major:
 *   grad_a [m, k] = grad . b^T      grad_b [k, n] = a^T . grad
 * Either output may be NULL (not computed).  Two gfh_sgemm launches (NT and
 * TN) on the stream. */
GFH_API int gfh_matmul_backward_f32(const float *grad, const float *a, const float *b,
                                    int64_t m, int64_t k, int64_t n, float *grad_a,
                                    float *grad_b, gfh_stream_t stream);

/* ---- int8 quantization (ghostflow-nn/src/quantization.rs) ---------------- */

/* quantize_per_channel_int8 (quantization.rs:110-153): channel = dim 0, one
 * (scale, zero_point) per contiguous row of `cols` elements; symmetric or
 * asymmetric.  Codes, scales and zero points are bit-identical to the
 * reference. */
GFH_API int gfh_quantize_i8_per_channel(const float *x, int64_t rows, int64_t cols,
                                        int symmetric, int8_t *q, float *scales,
                                        int8_t *zero_points, gfh_stream_t stream);

/* quantize_per_tensor_int8 (quantization.rs:77-108): one (scale, zero_point)
 * over all n elements; DynamicQuantization::quantize_activation uses it with
 * symmetric = 0 (quantization.rs:280-287).  `scale` / `zero_point` are device
 * pointers to one element each.  Workspace: gfh_quantize_i8_per_tensor_
 * workspace_size(n) bytes (nullable, see conventions). */
GFH_API int gfh_quantize_i8_per_tensor(const float *x, int64_t n, int symmetric,
                                       int8_t *q, float *scale, int8_t *zero_point,
                                       void *workspace, size_t workspace_bytes,
                                       gfh_stream_t stream);
GFH_API size_t gfh_quantize_i8_per_tensor_workspace_size(int64_t n);

/* dequantize_int8 (quantization.rs:173-204): nscales == 1 -> per tensor,
 * nscales == rows -> per channel over dim 0; (q - zp) * scale. */
GFH_API int gfh_dequantize_i8(const int8_t *q, int64_t rows, int64_t cols,
                              const float *scales, const int8_t *zero_points,
                              int64_t nscales, float *out, gfh_stream_t stream);

/* Sum over k of qw[n, k] for every row n (int32), the zero-point correction
 * term of gfh_qlinear_i8.  Weights are static, so this runs once per weight. */
GFH_API int gfh_qweight_rowsum(const int8_t *qw, int64_t n, int64_t k,
                               int32_t *rowsum, gfh_stream_t stream);

/* INT8 linear.  The reference has no integer GEMM (its executable path is
 * DynamicQuantization::get_weights -> dequantize -> fp32 matmul,
 * quantization.rs:275-277); this computes the same layer on int8 MFMA:
 *   acc[m,n] = sum_k (qx[m,k] - zx) * qw[n,k]          exact int32
 *            = sum_k qx*qw - zx * rowsum[n]
 *   y[m,n]   = (float)acc * (sx * sw[n]) (+ bias[n])   each step f32-rounded
 * x_per_row = 0: sx, zx point to ONE element (per-tensor activation,
 *   quantization.rs:280-287);  x_per_row = 1: sx[m], zx[m] per row
 *   (QuantizationConfig::default, per-channel over dim 0, :28-36).
 * zx and w_rowsum are nullable (zero points taken as 0; w_rowsum is required
 * when zx is given).  qw is [n, k] with per-row scales sw[n]
 * (quantize_per_channel_int8 of the Linear weight [out, in]).
 * y and acc_out are nullable (at least one must be given); acc_out receives
 * the exact int32 accumulators. */
GFH_API int gfh_qlinear_i8(const int8_t *qx, const float *sx, const int8_t *zx,
                           int x_per_row, const int8_t *qw, const float *sw,
                           const int32_t *w_rowsum, const float *bias, float *y,
                           int32_t *acc_out, int64_t m, int64_t n, int64_t k,
                           gfh_stream_t stream);

/* The same layer on fp32 activations x [m, k]: DynamicQuantization::
 * quantize_activation (per tensor, asymmetric, quantization.rs:280-287) of x
 * followed by gfh_qlinear_i8 with x_per_row = 0.  The codes, and so y, are
 * exactly those of gfh_quantize_i8_per_tensor(symmetric = 0) followed by
 * gfh_qlinear_i8.  For m <= 4 (k % 16 == 0, aligned x and qw) it is one
 * launch: every workgroup finds the min / max of x and quantizes its part
 * itself, and no workspace is used.  Otherwise the quantize pass writes the
 * codes to workspace (nullable; at least
 * gfh_qlinear_dynamic_i8_workspace_size(m, k) bytes, 16-byte aligned).
 * w_rowsum is required. */
GFH_API size_t gfh_qlinear_dynamic_i8_workspace_size(int64_t m, int64_t k);
GFH_API int gfh_qlinear_dynamic_i8(const float *x, const int8_t *qw, const float *sw,
                                   const int32_t *w_rowsum, const float *bias, float *y,
                                   int64_t m, int64_t n, int64_t k, void *workspace,
                                   size_t workspace_bytes, gfh_stream_t stream);

/* ---- decode GEMV --------------------------------------------------------- */

/* y[b, n] = sum_k x[b, k] * W[k, n], W [k, n] row-major, b <= 64.
 * Tensor::matmul with M = b (matmul.rs:91-119); Tensor::mv for b = 1
 * (matmul.rs:222-250). */
GFH_API int gfh_gemv_f32(const float *x, const float *w, float *y, int64_t b,
                         int64_t k, int64_t n, gfh_stream_t stream);

/* Weight-only int8 GEMV: W is QuantizedTensor data [k, n] quantized per
 * channel over dim 0 (quantize_per_channel_int8, quantization.rs:110-153), so
 * row k has scale s[k] and zero point zp[k] (zp nullable = 0):
 *   y[b, n] = sum_k x[b, k] * ((q[k, n] - zp[k]) * s[k])
 * i.e. DynamicQuantization::get_weights (dequantize_int8, :173-204) followed
 * by Tensor::matmul, without materializing the fp32 weight. b <= 64.
 * Precision: the products are regrouped as (x[b, k] * s[k]) * (q - zp).  Per
 * K-slice of up to 1024 rows, x * s is scaled by a power of two so that its
 * largest finite magnitude lies in [2^14, 2^15), then carried as three f16
 * (hi + mid + lo: 33 significant bits, so every fp32 x * s down to 2^-16
 * times the slice maximum is carried exactly; smaller values keep an
 * absolute error under 2^-39 times that maximum, f16's subnormal step).  The
 * products are exact and summed in fp32, so y stays within the fp32 GEMM
 * bound of the reference but is not bit-identical to it.  An infinite or
 * NaN x * s is carried unchanged and gives inf / NaN as the reference does. */
GFH_API int gfh_gemv_w8(const float *x, const int8_t *qw, const float *scales,
                        const int8_t *zero_points, float *y, int64_t b,
                        int64_t k, int64_t n, gfh_stream_t stream);

/* Allocation-free gfh_gemv_w8.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments, kernels and results as gfh_gemv_w8 (bit for bit); it calls no
 * hipMalloc / hipFree / allocating library routine.  Its split-K partials
 * and arrival counters live in a static device array of 8 MiB + 64 KiB that
 * each GPU holds until the process ends.  Limit: a call whose K is split
 * needs 4 * slices * min(b, 8) * n bytes of partials (at most 8 MiB) and
 * ceil(n / 256) counters (at most 16384); larger calls return
 * GFH_INVALID_SHAPE before launching anything.  (W [4096, 14336] at b = 8
 * needs 1.8 MiB; W [11008, 4096]-shaped [4096, 11008] at b = 8, 2.8 MiB.)
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialized by the caller. */
GFH_API int gfh_gemv_w8_noalloc(const float *x, const int8_t *qw,
                                const float *scales, const int8_t *zero_points,
                                float *y, int64_t b, int64_t k, int64_t n,
                                gfh_stream_t stream);

/* ---- attention ----------------------------------------------------------- */

/* Row softmax over the last dimension (Tensor::softmax(-1),
 * ghostflow-core/src/ops/activation.rs:165-216).  x and y may alias. */
GFH_API int gfh_softmax_lastdim_f32(const float *x, float *y, int64_t rows,
                                    int64_t cols, gfh_stream_t stream);

/* Fused scaled-dot-product attention, Q [b,h,sq,d], K/V [b,h,skv,d],
 * out [b,h,sq,d]:  softmax(mask(Q.K^T * scale)) . V
 *   - scale multiplies the finished dot product (mul_scalar after the
 *     matmul, ghostflow-nn/src/attention.rs:19-25);
 *   - causal != 0 masks j > i (ghostflow-cuda/src/ops.rs:205-224; needs
 *     sq == skv);
 *   - mask (nullable, f32, mask_numel elements) is CYCLED over the flattened
 *     scores, m > 0.5 keeps (apply_attention_mask, attention.rs:51-64);
 *   - weights (nullable) receives the [b,h,sq,skv] softmax output, the
 *     second value scaled_dot_product_attention returns (attention.rs:48).
 * Replaces scaled_dot_product_attention (attention.rs:11-49),
 * ops::attention::flash_attention (ghostflow-cuda/src/ops.rs:166-203) and
 * launch_fused_attention (ghostflow-cuda/src/ffi.rs:190-196).  d <= 128 and
 * d % 4 == 0. */
GFH_API int gfh_sdpa_f32(const float *q, const float *k, const float *v, float *out,
                         float *weights, int64_t b, int64_t h, int64_t sq,
                         int64_t skv, int64_t d, float scale, int causal,
                         const float *mask, int64_t mask_numel, gfh_stream_t stream);

/* FlashAttention::forward (ghostflow-nn/src/flash_attention.rs:81-250) with
 * FlashAttentionConfig's block_size_m / block_size_n / causal / scale
 * (:14-68; dropout is not applied by the reference's forward): q [batch,
 * seq_len_q, d_model], k / v [batch, seq_len_k, d_model], out [batch,
 * seq_len_q, d_model].  The reference's own blockwise recurrence, as it is:
 *   - causal masks key j for query i when j > i (absolute indices, top-left
 *     aligned also when seq_len_q != seq_len_k, :193-196), and skips key
 *     blocks that start at or past the end of the query block (:150-152);
 *   - the running-max correction exp(old_max - new_max) multiplies the
 *     output once per KEY of each block (:233-241), so the result is not
 *     softmax attention unless block_size_n == 1: the first key block keeps
 *     only its last key, and a block whose max rises scales the earlier
 *     output by the correction to the power of its key count;
 *   - rows with row_sum == 0 are left undivided (:166-172); no keys gives 0.
 * Within fp32 rounding of the reference (1e-4 relative) for finite inputs;
 * the block maxima are exact (fp64 scores of their keys), so the result is
 * nearer the exact value of the recurrence than the reference's own fp32
 * evaluation.  Block sizes must be positive (the reference's step_by(0)
 * panics) and ceil(seq_len_k / block_size_n) <= 8192.  Workspace:
 * gfh_flash_attention_workspace_size(batch, seq_len_q, seq_len_k) bytes,
 * 8-byte aligned (nullable, see conventions).  For softmax attention use
 * gfh_sdpa_f32. */
GFH_API int gfh_flash_attention_f32(const float *q, const float *k, const float *v,
                                    float *out, int64_t batch, int64_t seq_len_q,
                                    int64_t seq_len_k, int64_t d_model,
                                    int64_t block_size_m, int64_t block_size_n,
                                    int causal, float scale, void *workspace,
                                    size_t workspace_bytes, gfh_stream_t stream);
GFH_API size_t gfh_flash_attention_workspace_size(int64_t batch, int64_t seq_len_q,
                                                  int64_t seq_len_k);

/* Attention of sq new queries over a key/value cache, in the reference's
 * [B, S, E] layout with head hh in columns hh*d .. hh*d+d-1 (the storage of
 * reshape_for_attention's [B, H, S, D] view, ghostflow-nn/src/attention.rs:
 * 146-150):
 *   q      [b, sq, ldq]           projected queries
 *   k, v   [b, capacity, ldkv]    cache rows [0, kv_len) are attended to
 *   out    [b, sq, ldo]           heads merged (reshape_from_attention, :152-157)
 *   weights (nullable)            [b, h, sq, kv_len] softmax probabilities
 * per (b, hh): softmax(mask(q . k^T * scale)) . v -- the
 * scaled_dot_product_attention step (:11-49) of
 * MultiHeadAttention::forward_with_cache (:100-144), reading the cache in
 * place where the reference concatenates past and new keys (concat_tensors,
 * :214-247).  mask (nullable) is cycled over the flattened
 * [b, h, sq, kv_len] scores, m > 0.5 keeps (:51-64); causal != 0 keeps key j
 * for query i when j <= kv_len - sq + i (needs kv_len >= sq).  A query with
 * every key masked gets NaN, as in the reference.  d % 4 == 0, d <= 128;
 * ldq, ldkv, ldo multiples of 4 and >= h*d; q, k, v, out 16-byte aligned.
 * Meant for few queries (decode); long query runs are better served by
 * gfh_sdpa_f32. */
GFH_API int gfh_kv_attention_f32(const float *q, int64_t ldq, const float *k,
                                 const float *v, int64_t capacity, int64_t ldkv,
                                 float *out, int64_t ldo, float *weights, int64_t b,
                                 int64_t h, int64_t sq, int64_t kv_len, int64_t d,
                                 float scale, int causal, const float *mask,
                                 int64_t mask_numel, gfh_stream_t stream);

/* ---- multi-head attention with a key/value cache ------------------------ */

/* MultiHeadAttention::forward_with_cache (ghostflow-nn/src/attention.rs:
 * 100-144) with dropout off, on an in-place K/V cache:
 *   query [b, sq, e], key / value [b, sk, e];
 *   wq, wk, wv, wo [e, e] as Linear weights [out, in]; biases [e] nullable;
 *   k_cache, v_cache [b, capacity, e]: rows [0, past_len) hold the earlier
 *     projected keys/values (the reference's past_key / past_value); this
 *     call writes key . Wk^T + bk and value . Wv^T + bv into rows
 *     [past_len, past_len + sk) -- the concatenation along dim 1 of
 *     concat_tensors (:214-247) without the copy, and the new k/v the
 *     reference returns (:141-142, in [b, sk, e] storage order);
 *   out [b, sq, e] = out_proj(attention(q, k_cache, v_cache));
 *   weights (nullable) [b, h, sq, past_len + sk] softmax probabilities.
 * scale = 1 / sqrt(e / h) (attention.rs:19-20); mask (nullable) is cycled
 * over the flattened [b, h, sq, past_len + sk] scores (:51-64); causal != 0
 * keeps key j for query i when j <= past_len + sk - sq + i, which equals
 * passing the matching lower-triangular mask.  e / h must be a multiple of
 * 4 in [4, 128]; k_cache and v_cache 16-byte aligned.  workspace (nullable,
 * 16-byte aligned) of at least gfh_mha_workspace_size(b, sq, e) bytes holds
 * the projected queries and the attention output; without one the call
 * allocates stream-ordered. */
GFH_API size_t gfh_mha_workspace_size(int64_t b, int64_t sq, int64_t e);
GFH_API int gfh_mha_forward_with_cache_f32(
    const float *query, const float *key, const float *value, const float *wq,
    const float *bq, const float *wk, const float *bk, const float *wv,
    const float *bv, const float *wo, const float *bo, float *k_cache,
    float *v_cache, int64_t capacity, int64_t past_len, const float *mask,
    int64_t mask_numel, int causal, float *out, float *weights, int64_t b,
    int64_t sq, int64_t sk, int64_t e, int64_t h, void *workspace,
    size_t workspace_bytes, gfh_stream_t stream);

/* ---- SwiGLU feed-forward block ------------------------------------------ */

/* out[i] = silu(gate[i]) * up[i], silu(v) = v / (1 + exp(-v)): the
 * gate.silu().mul(&up) step of SwiGLU::forward (ghostflow-nn/src/llama.rs:
 * 281-283; silu = ghostflow-core/src/ops/activation.rs:117-122, mul =
 * arithmetic.rs:39-45).  out may alias gate or up. */
GFH_API int gfh_silu_mul_f32(const float *gate, const float *up, float *out, int64_t n,
                             gfh_stream_t stream);

/* SwiGLU::forward (ghostflow-nn/src/llama.rs:276-286), fp32:
 *   y = (silu(x . Wg^T + bg) * (x . Wu^T + bu)) . Wd^T + bd
 * x [m, hidden]; wg, wu [inter, hidden] and wd [hidden, inter] as Linear
 * weights [out, in]; biases nullable (Linear::new has them, linear.rs:18-20);
 * y [m, hidden]; h (nullable) [m, inter] receives silu(gate) * up.
 * workspace (nullable, 16-byte aligned) of at least
 * gfh_swiglu_f32_workspace_size(m, inter) bytes; without one the call
 * allocates stream-ordered. */
GFH_API size_t gfh_swiglu_f32_workspace_size(int64_t m, int64_t inter);
GFH_API int gfh_swiglu_f32(const float *x, int64_t m, int64_t hidden, int64_t inter,
                           const float *wg, const float *bg, const float *wu, const float *bu,
                           const float *wd, const float *bd, float *y, float *h,
                           void *workspace, size_t workspace_bytes, gfh_stream_t stream);

/* SwiGLU::forward with each Linear as the INT8 linear (gfh_qlinear_i8) on
 * DynamicQuantization's scheme (ghostflow-nn/src/quantization.rs:251-288):
 *   qwg, qwu [inter, hidden], qwd [hidden, inter]: per-channel symmetric
 *     codes (quantize_per_channel_int8, :110-153) with scales swg / swu /
 *     swd and row sums rsg / rsu / rsd (gfh_qweight_rowsum);
 *   x and h = silu(gate) * up are quantized per tensor, asymmetric
 *     (quantize_activation, :280-287) on the device;
 *   gate, up and y are the dequantized fp32 outputs plus bias.
 * h (nullable) [m, inter] receives silu(gate) * up.  workspace (nullable,
 * 16-byte aligned) of at least gfh_swiglu_i8_workspace_size(m, hidden,
 * inter) bytes.  hidden and inter must be multiples of 16. */
GFH_API size_t gfh_swiglu_i8_workspace_size(int64_t m, int64_t hidden, int64_t inter);
GFH_API int gfh_swiglu_i8(const float *x, int64_t m, int64_t hidden, int64_t inter,
                          const int8_t *qwg, const float *swg, const int32_t *rsg,
                          const float *bg, const int8_t *qwu, const float *swu,
                          const int32_t *rsu, const float *bu, const int8_t *qwd,
                          const float *swd, const int32_t *rsd, const float *bd, float *y,
                          float *h, void *workspace, size_t workspace_bytes,
                          gfh_stream_t stream);

/* ---- state dict files (ghostflow-core/src/serialize.rs) ------------------ */

/* An opened weight file, mapped into host memory.  Two formats:
 *
 * GHOSTFLW -- the reference's state dict (serialize.rs:11-186):
 *   "GHOSTFLW" | u32 version (1) | u32 count | count x entry, where an entry
 *   is u32 name length | UTF-8 name | u8 dtype (serialize.rs:188-215:
 *   0 F16 .. 2 F32 .. 9 Bool) | u32 ndim | ndim x u64 dims | numel x f32;
 *   every integer and float little-endian, the data always f32 whatever the
 *   dtype byte says (write_tensor uses data_f32).
 *
 * GHOSTFLQ -- this library's file for QuantizedTensor
 *   (ghostflow-nn/src/quantization.rs:40-51), which the reference cannot
 *   write; payloads start at 64-byte file offsets:
 *   "GHOSTFLQ" | u32 version (1) | u32 count | count x entry, an entry being
 *   u32 name length | UTF-8 name | u8 kind, then
 *     kind 0 (f32 tensor): u8 dtype | u32 ndim | u64 dims | pad | numel x f32
 *     kind 1 (QuantizedTensor): u8 scheme (QuantizationScheme order: 0 INT8,
 *       1 FP16, 2 Dynamic) | u32 ndim | u64 dims | u64 nscales (1: per
 *       tensor, dims[0]: per channel over dim 0) | pad | nscales x f32
 *       scales | nscales x i8 zero points | pad | numel x i8 codes
 *
 * Opening validates the file the way load_state_dict does (serialize.rs:
 * 47-88, 122-167): magic, version <= 1, dtype byte 0-9, UTF-8 names, every
 * size inside the file; errors are GFH_INVALID_DATA with the reason in
 * gfh_last_error().  A name stored twice keeps its last entry, as the
 * reference's HashMap insert does.  The handle owns the mapping and the
 * pinned staging buffers; it is not thread-safe. */
typedef struct gfh_state_dict gfh_state_dict;
GFH_API int gfh_state_dict_open(const char *path, gfh_state_dict **out);
GFH_API void gfh_state_dict_close(gfh_state_dict *sd);
/* Number of distinct names. */
GFH_API int64_t gfh_state_dict_count(const gfh_state_dict *sd);
/* Entry `index` (0 .. count-1, in order of first appearance): name (valid
 * until close), kind (0 f32, 1 quantized), dtype byte (kind 0) or scheme
 * (kind 1), ndim, the first max_dims dims, nscales (kind 1; 0 otherwise).
 * Any output pointer may be NULL. */
GFH_API int gfh_state_dict_entry(const gfh_state_dict *sd, int64_t index, const char **name,
                                 int *kind, int *dtype, int *ndim, int64_t *dims, int max_dims,
                                 int64_t *nscales);
/* Index of `name`, or -1. */
GFH_API int64_t gfh_state_dict_find(const gfh_state_dict *sd, const char *name);
/* Copy an entry into device memory: a kind-0 entry's numel floats into dst;
 * a kind-1 entry's codes, scales and zero points.  The copies run on
 * `stream` through pinned staging buffers; the call returns once the data
 * is in device memory. */
GFH_API int gfh_state_dict_read_f32(gfh_state_dict *sd, int64_t index, float *dst,
                                    gfh_stream_t stream);
GFH_API int gfh_state_dict_read_q8(gfh_state_dict *sd, int64_t index, int8_t *codes,
                                   float *scales, int8_t *zero_points, gfh_stream_t stream);

/* One tensor to write; pointers marked device are device memory. */
typedef struct gfh_tensor_entry {
    const char *name;
    int kind;                   /* 0 f32 tensor, 1 QuantizedTensor (GHOSTFLQ only) */
    int dtype;                  /* kind 0: dtype byte to record (2 = F32); kind 1: scheme */
    int ndim;
    const int64_t *dims;        /* host, ndim entries */
    const void *data;           /* device: numel f32 (kind 0) or numel int8 codes (kind 1) */
    const float *scales;        /* device, kind 1: nscales */
    const int8_t *zero_points;  /* device, kind 1: nscales */
    int64_t nscales;            /* kind 1: 1 or dims[0] */
} gfh_tensor_entry;
/* save_state_dict (serialize.rs:20-45) from device memory: a GHOSTFLW file
 * (quantized_format == 0; kind-0 entries only, in the given order, byte for
 * byte what write_tensor writes) or a GHOSTFLQ file.  Waits for `stream`
 * before reading the tensors. */
GFH_API int gfh_state_dict_save(const char *path, int quantized_format,
                                const gfh_tensor_entry *entries, int64_t count,
                                gfh_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GHOSTFLOW_HIP_H */
