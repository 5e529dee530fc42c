// kernels.hpp -- host-side launchers of the gfx950 kernels.  Arguments are
// validated by the C ABI layer (api.hip) before any of these is called.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gfh {

struct SgemmDesc {
    bool trans_a = false, trans_b = false;
    int64_t m = 0, n = 0, k = 0;
    float alpha = 1.f, beta = 0.f;
    const float *a = nullptr;
    int64_t lda = 0, stride_a = 0, batch_a = 1;
    const float *b = nullptr;
    int64_t ldb = 0, stride_b = 0, batch_b = 1;
    float *c = nullptr;
    int64_t ldc = 0, stride_c = 0;
    int64_t batch = 1;
    const float *bias = nullptr;
};
int launch_sgemm(const SgemmDesc &d, hipStream_t s);
// gemv_nt.hip: the NT form at m <= kNtSkinnyMinM (Linear at decode sizes);
// launch_sgemm uses it when gemv_nt_fits.  The grouped form runs up to
// kNtMaxGroups unbatched NT products of one shape (m, n, k, lda, ldb, alpha,
// beta) with their own operands, bias and ldc in one launch.
bool gemv_nt_fits(const SgemmDesc &d);
int launch_gemv_nt(const SgemmDesc &d, hipStream_t s);
constexpr int kNtMaxGroups = 3;
bool gemv_nt_group_fits(const SgemmDesc *d, int count);
int launch_gemv_nt_group(const SgemmDesc *d, int count, hipStream_t s);
// gemm_nt_skinny.hip: the NT form at kNtSkinnyMinM < m <= 64 on f32 MFMA
// with the weight streamed into registers; launch_sgemm uses it when
// gemm_nt_skinny_fits.  Grouped like the row-dot form.
constexpr int64_t kNtSkinnyMinM = 4;
bool gemm_nt_skinny_fits(const SgemmDesc &d);
int launch_gemm_nt_skinny(const SgemmDesc &d, hipStream_t s);
bool gemm_nt_skinny_group_fits(const SgemmDesc *d, int count);
int launch_gemm_nt_skinny_group(const SgemmDesc *d, int count, hipStream_t s);
// sgemm.hip: up to kNtMaxGroups NT products of one shape at m <= 64 in one
// launch (whichever of the two forms above serves m), or false / an error
// when they do not fit one.
bool sgemm_nt_group_fits(const SgemmDesc *d, int count);
int launch_sgemm_nt_group(const SgemmDesc *d, int count, hipStream_t s);
// sgemm_big.hip: NT and NN (A [m, k]) on direct-to-LDS tiles -- 256 x 256 or
// 128 x 128 when they fill the GPU, else 64 x 64 (K % 32 == 0, batch 1; NN
// with n % 4 == 0).
bool sgemm_big_fits(const SgemmDesc &d);
int launch_sgemm_big(const SgemmDesc &d, hipStream_t s);

// quant.hip
int launch_quantize_per_channel(const float *x, int64_t rows, int64_t cols, bool symmetric, int8_t *q,
                                float *scales, int8_t *zps, hipStream_t s);
size_t quantize_per_tensor_workspace(int64_t n);
int launch_quantize_per_tensor(const float *x, int64_t n, bool symmetric, int8_t *q, float *scale, int8_t *zp,
                               void *ws, hipStream_t s);
int launch_quantize_per_tensor_partials(const float *x, int64_t n, bool symmetric, const float2 *partials,
                                       int npartials, int8_t *q, float *scale, int8_t *zp, hipStream_t s);
int launch_dequantize(const int8_t *q, int64_t rows, int64_t cols, const float *scales, const int8_t *zps,
                      int64_t nscales, float *out, hipStream_t s);
int launch_rowsum_i8(const int8_t *q, int64_t n, int64_t k, int32_t *rowsum, hipStream_t s);

// qgemm.hip
struct QLinearDesc {
    const int8_t *qx = nullptr;
    const float *sx = nullptr;
    const int8_t *zx = nullptr;
    bool x_per_row = false;
    const int8_t *qw = nullptr;
    const float *sw = nullptr;
    const int32_t *w_rowsum = nullptr;
    const float *bias = nullptr;
    float *y = nullptr;
    int32_t *acc = nullptr;
    int64_t m = 0, n = 0, k = 0;
    // In place of qx / sx / zx: fp32 activations [m, k] that the kernel
    // quantizes itself, per tensor and asymmetric, from the (min, max) of all
    // of them or of the nxpart partials xpart (a producer's); only where
    // qlinear_qx_fits (m <= 4 and few codes per workgroup).
    const float *xf = nullptr;
    const float2 *xpart = nullptr;
    int nxpart = 0;
};
bool qlinear_qx_fits(int64_t m, int64_t n, int64_t k, bool partials);
int launch_qlinear_i8(const QLinearDesc &d, hipStream_t s);
// SwiGLU gate/up in one launch: h = silu(x.Wg^T + bg) * (x.Wu^T + bu) with x
// quantized per tensor (g.zx per tensor, g.x_per_row false); g carries x,
// the gate weight and h (as y), the up_* fields the up weight.  Writes one
// (min, max) of h per workgroup into hpart and their count into *npart.
struct QSwigluDesc {
    QLinearDesc g;
    const int8_t *qw_up = nullptr;
    const float *sw_up = nullptr;
    const int32_t *rowsum_up = nullptr;
    const float *bias_up = nullptr;
    float2 *hpart = nullptr;
};
// Whether the fused launch serves this shape (else: two INT8 linears and
// launch_silu_mul), and the hpart capacity it needs.
bool qlinear_swiglu_fits(int64_t m, int64_t n, int64_t k);
int64_t qlinear_swiglu_partials(int64_t m, int64_t n);
int launch_qlinear_swiglu_i8(const QSwigluDesc &d, int *npart, hipStream_t s);

// gemv.hip
int launch_gemv_f32(const float *x, const float *w, float *y, int64_t b, int64_t k, int64_t n, hipStream_t s);
// The same with gfh_sgemm's epilogue: y = alpha * (x . W) (+ beta * y) (+ bias),
// each a separately rounded f32 operation.
int launch_gemv_f32_epi(const float *x, const float *w, float *y, int64_t b, int64_t k, int64_t n, float alpha,
                        float beta, const float *bias, hipStream_t s);
int launch_gemv_w8(const float *x, const int8_t *qw, const float *scales, const int8_t *zps, float *y, int64_t b,
                   int64_t k, int64_t n, hipStream_t s);
// Same computation with its split-K scratch in a static device array: no
// allocation.  Sizes beyond that array are rejected before any launch.
int launch_gemv_w8_noalloc(const float *x, const int8_t *qw, const float *scales, const int8_t *zps, float *y,
                           int64_t b, int64_t k, int64_t n, hipStream_t s);

// flash_attention.hip: FlashAttention::forward (blockwise recurrence) as
// scores GEMM -> per-row weights kernel -> weights . V GEMM; ws holds
// batch * sq * sk floats.
struct FlashAttnDesc {
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    float *out = nullptr;
    float *ws = nullptr;
    int64_t batch = 0, sq = 0, sk = 0, d = 0, block_m = 64, block_n = 64;
    bool causal = false;
    float scale = 1.f;
};
int64_t flash_attention_max_blocks();
// Scratch the launch needs in d.ws: the per-row block maxima of the fused
// form, or the [batch, sq, sk] scores of the three-step form.
size_t flash_attention_workspace_bytes(const FlashAttnDesc &d);
int launch_flash_attention_blockwise(const FlashAttnDesc &d, hipStream_t s);

// attention.hip
int launch_softmax_lastdim(const float *x, float *y, int64_t rows, int64_t cols, hipStream_t s);
struct SdpaDesc {
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    float *out = nullptr;
    float *weights = nullptr;
    int64_t b = 0, h = 0, sq = 0, skv = 0, d = 0;
    float scale = 1.f;
    bool causal = false;
    const float *mask = nullptr;
    int64_t mask_numel = 0;
    // Element strides (b, h, row) of q, k/v and out when `strided`;
    // otherwise [b, h, s, d] contiguous.  causal keeps key j for query i
    // when j <= i + skv - sq.
    bool strided = false;
    int64_t q_bs = 0, q_hs = 0, q_rs = 0, kv_bs = 0, kv_hs = 0, kv_rs = 0, o_bs = 0, o_hs = 0, o_rs = 0;
};
int launch_sdpa(const SdpaDesc &d, hipStream_t s);

// kv_attention.hip: a few queries over a K/V cache in [B, S, E] layout
// (head h in columns h*d ..); strides in elements.
struct KvAttnDesc {
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    float *out = nullptr;
    float *weights = nullptr;  // [b, h, sq, kv_len], nullable
    const float *mask = nullptr;
    int64_t mask_numel = 0;
    int64_t q_bs = 0, q_rs = 0, kv_bs = 0, kv_rs = 0, o_bs = 0, o_rs = 0;
    int64_t b = 0, h = 0, sq = 0, kv_len = 0, d = 0;
    float scale = 1.f;
    bool causal = false;
};
int launch_kv_attention(const KvAttnDesc &d, hipStream_t s);

// mha.hip: MultiHeadAttention::forward_with_cache over a [b, capacity, e]
// K/V cache; the workspace holds the projected queries and the attention
// output (mha_workspace_bytes).
struct MhaDesc {
    const float *query = nullptr, *key = nullptr, *value = nullptr;
    const float *wq = nullptr, *bq = nullptr, *wk = nullptr, *bk = nullptr;
    const float *wv = nullptr, *bv = nullptr, *wo = nullptr, *bo = nullptr;
    float *k_cache = nullptr, *v_cache = nullptr;
    int64_t capacity = 0, past_len = 0;
    const float *mask = nullptr;
    int64_t mask_numel = 0;
    bool causal = false;
    float *out = nullptr, *weights = nullptr;
    int64_t b = 0, sq = 0, sk = 0, e = 0, h = 0;
    float scale = 1.f;
};
size_t mha_workspace_bytes(int64_t b, int64_t sq, int64_t e);
int launch_mha_forward(const MhaDesc &d, void *workspace, hipStream_t s);

// swiglu.hip: SwiGLU::forward (llama.rs:276-286).  x [m, hidden]; gate / up
// weights [inter, hidden], down weight [hidden, inter] (Linear [out, in]);
// biases nullable; h (nullable) receives silu(gate) * up [m, inter].
struct SwigluDesc {
    const float *x = nullptr;
    int64_t m = 0, hidden = 0, inter = 0;
    const float *wg = nullptr, *bg = nullptr, *wu = nullptr, *bu = nullptr, *wd = nullptr, *bd = nullptr;
    const int8_t *qwg = nullptr, *qwu = nullptr, *qwd = nullptr;
    const float *swg = nullptr, *swu = nullptr, *swd = nullptr;
    const int32_t *rsg = nullptr, *rsu = nullptr, *rsd = nullptr;
    float *y = nullptr, *h = nullptr;
};
int launch_silu_mul(const float *g, const float *u, float *out, int64_t n, hipStream_t s);
size_t swiglu_f32_workspace_bytes(int64_t m, int64_t inter);
int launch_swiglu_f32(const SwigluDesc &d, void *workspace, hipStream_t s);
size_t swiglu_i8_workspace_bytes(int64_t m, int64_t hidden, int64_t inter);
int launch_swiglu_i8(const SwigluDesc &d, void *workspace, hipStream_t s);

}  // namespace gfh
