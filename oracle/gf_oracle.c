/*
 * gf_oracle.c -- CPU restatement of GhostFlow's dense hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP library is
 * compared against; it is never linked into, loaded by or called from the
 * product library.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may use it.
 *
 * The reference (choksi2212/ghost-flow) is Rust and cannot be built in this
 * image (no rustc/cargo, no crates.io), so each function below restates the
 * reference's algorithm step by step, citing the file:line it follows
 * (paths relative to the reference checkout).  Build flags
 * -O3 -ffp-contract=off -fno-fast-math -march=x86-64 keep every f32 `a*b`
 * and `c+p` a separately rounded IEEE operation, as rustc emits them (Rust
 * never contracts to FMA), so results are expected to be bit-identical to
 * the Rust build on the same host.
 *
 * Pinning (what checks each function; tests/test_oracle.py, and the
 * committed .npz fixtures under tests/golden/ that tests/test_golden.py
 * regenerates bit for bit):
 *   gfo_matmul_blocked / gfo_batched_matmul : reference known answers
 *       [[22,28],[49,64]] (matmul.rs:331-352) and [19,22,43,50]
 *       (tests/test_optimizations.rs:65-91); integer-valued inputs
 *       (exact in any order) against an int64 brute force; fp64 brute force
 *       error bound on random inputs; identity / permutation matrices.
 *   gfo_transpose_last2 : explicit index check against numpy transpose.
 *   gfo_matmul_backward : integer-valued inputs against int64 brute force
 *       (grad . b^T and a^T . grad); the sequential-order tie 2^24 + 1 + 1;
 *       fp64 brute force bound; finite-difference-free identity
 *       <grad, A.B> consistency with the forward.
 *   gfo_linear_forward  : integer-valued inputs against int64 brute force
 *       with bias; equals matmul(x, W^T) + b computed by the pinned parts.
 *   gfo_softmax_lastdim : rows sum to 1 (activation.rs:266-272,
 *       tests/test_optimizations.rs:51-62); constant row -> uniform;
 *       fp64 closed form within a few ulp; all -inf row -> NaN.
 *   gfo_silu_mul : silu(0) = 0, silu(x) = x once exp(-x) < ulp(1)/2,
 *       silu(-x) = -0 once exp(x) overflows; bit-exact against a float32
 *       restatement on inputs whose expf is unambiguous, chosen so that
 *       the plausible x * (1 / (1 + e)) form differs; fp64 closed form
 *       within a few ulp.
 *   gfo_sdpa / gfo_flash_attention : causal row 0 == V[0] exactly;
 *       constant K -> prefix mean of V; fp64 brute force on tiny shapes;
 *       cycled [S,S] causal mask == causal flag path bit for bit.
 *   gfo_quantize_per_tensor / _per_channel / gfo_dequantize : exact codes
 *       derived by hand from quantization.rs:77-153 for the reference's own
 *       test inputs (half-away-from-zero tie, zero-point saturation), the
 *       reference round-trip bounds (quantization.rs:300-428), and an
 *       exhaustive numpy restatement on random data.
 *   gfo_qlinear_i8 : int32 accumulator against an int64 brute force GEMM;
 *       epilogue against an fp64 evaluation of the same formula.
 *   gfo_broadcast_binary : the reference's own add tests ([1,2,3] + [4,5,6]
 *       = [5,7,9] and [3,1] + [1,2] -> [3,2], arithmetic.rs:257-271); numpy
 *       broadcasting (a single IEEE add / mul per element, so bit-exact) on
 *       stretched, prepended, scalar and zero-size shapes.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GFO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* Rust scalar semantics used by quantization.rs                             */
/* ------------------------------------------------------------------------ */

/* `f as i32`: NaN -> 0, saturate to [i32::MIN, i32::MAX]. */
static int32_t rust_f32_as_i32(float f) {
    if (isnan(f)) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

/* `f as i8`: NaN -> 0, saturate to [-128, 127]. */
static int8_t rust_f32_as_i8(float f) {
    if (isnan(f)) return 0;
    if (f >= 127.0f) return 127;
    if (f <= -128.0f) return -128;
    return (int8_t)f;
}

/* `a + b` on i32 in a release build (overflow-checks off): wrapping. */
static int32_t rust_wrapping_add_i32(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

/* ------------------------------------------------------------------------ */
/* ghostflow-core/src/ops/matmul.rs                                          */
/* ------------------------------------------------------------------------ */

/* matmul.rs:91-119 `matmul_blocked`: C starts at +0.0 (`vec![0.0f32; m*n]`),
 * then for each row i, column block jb (64), k block kb (64), kk, j:
 * `row[j] += a_ik * b[kk*n + j]` -- per element the k order is ascending and
 * every product and sum is rounded separately.  Single-threaded
 * (`chunks_mut`, :101). */
GFO_API void gfo_matmul_blocked(const float *a, const float *b, float *c,
                                size_t m, size_t k, size_t n) {
    const size_t BLOCK = 64;
    memset(c, 0, m * n * sizeof(float));
    for (size_t i = 0; i < m; ++i) {
        float *row = c + i * n;
        for (size_t jb = 0; jb < n; jb += BLOCK) {
            size_t j_end = jb + BLOCK < n ? jb + BLOCK : n;
            for (size_t kb = 0; kb < k; kb += BLOCK) {
                size_t k_end = kb + BLOCK < k ? kb + BLOCK : k;
                for (size_t kk = kb; kk < k_end; ++kk) {
                    float a_ik = a[i * k + kk];
                    const float *brow = b + kk * n;
                    for (size_t j = jb; j < j_end; ++j) {
                        float p = a_ik * brow[j];
                        row[j] = row[j] + p;
                    }
                }
            }
        }
    }
}

/* matmul.rs:122-170 `batched_matmul`: for every output batch index, the A and
 * B slices are taken MODULO each operand's batch product (:148-149), then a
 * naive i-j-k loop with `sum = 0.0; sum += a*b` (ascending k). */
GFO_API void gfo_batched_matmul(const float *a, size_t a_batch,
                                const float *b, size_t b_batch,
                                float *c, size_t batch,
                                size_t m, size_t k, size_t n) {
    size_t ab = a_batch ? a_batch : 1, bb = b_batch ? b_batch : 1;
    for (size_t bi = 0; bi < batch; ++bi) {
        const float *as = a + (bi % ab) * m * k;
        const float *bs = b + (bi % bb) * k * n;
        float *cs = c + bi * m * n;
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < n; ++j) {
                float sum = 0.0f;
                for (size_t kk = 0; kk < k; ++kk) {
                    float p = as[i * k + kk] * bs[kk * n + j];
                    sum = sum + p;
                }
                cs[i * n + j] = sum;
            }
    }
}

/* ------------------------------------------------------------------------ */
/* ghostflow-core/src/ops/arithmetic.rs                                      */
/* ------------------------------------------------------------------------ */

/* arithmetic.rs:123-200 `broadcast_binary_op` for op 0 = add (x + y,
 * :20-26) and op 1 = mul (x * y, :39-45).  The caller passes the result
 * dims of Shape::broadcast_with (shape.rs:49-80).  Same shapes: element by
 * element (:141-154).  Otherwise each operand gets the strides of
 * compute_broadcast_strides (:180-201): walking its dims from the last,
 * stride = running product where its dim equals the result's (aligned at
 * the trailing dim), 0 where it is stretched; and flat index i of the
 * result is split innermost-first by compute_broadcast_index (:204-215). */
GFO_API void gfo_broadcast_binary(int op, const float *a, const size_t *a_dims, size_t a_nd,
                                  const float *b, const size_t *b_dims, size_t b_nd,
                                  float *c, const size_t *c_dims, size_t c_nd) {
    size_t numel = 1;
    for (size_t i = 0; i < c_nd; ++i) numel *= c_dims[i];
    int same = a_nd == b_nd;
    for (size_t i = 0; same && i < a_nd; ++i) same = a_dims[i] == b_dims[i];
    if (same) {
        for (size_t i = 0; i < numel; ++i) c[i] = op == 0 ? a[i] + b[i] : a[i] * b[i];
        return;
    }
    size_t *sa = calloc(c_nd ? c_nd : 1, sizeof(size_t)), *sb = calloc(c_nd ? c_nd : 1, sizeof(size_t));
    for (int w = 0; w < 2; ++w) {
        const size_t *dims = w ? b_dims : a_dims, nd = w ? b_nd : a_nd, off = c_nd - nd;
        size_t *st = w ? sb : sa, stride = 1;
        for (size_t i = nd; i-- > 0;) {
            if (dims[i] == c_dims[i + off]) {
                st[i + off] = stride;
                stride *= dims[i];
            } else {
                st[i + off] = 0;
            }
        }
    }
    for (size_t i = 0; i < numel; ++i) {
        size_t ia = 0, ib = 0, rem = i;
        for (size_t d = c_nd; d-- > 0;) {
            size_t coord = rem % c_dims[d];
            rem /= c_dims[d];
            ia += coord * sa[d];
            ib += coord * sb[d];
        }
        c[i] = op == 0 ? a[ia] + b[ib] : a[ia] * b[ib];
    }
    free(sa);
    free(sb);
}

/* ------------------------------------------------------------------------ */
/* ghostflow-core/src/tensor.rs                                              */
/* ------------------------------------------------------------------------ */

/* tensor.rs:318-340 `transpose(d-2, d-1)` is a stride swap; data_f32 on that
 * view (tensor.rs:223-279, `to_contiguous_data` + `for_each_index`) walks the
 * logical row-major order of the view, which for the last two dims is
 * out[b][j][i] = in[b][i][j]. */
GFO_API void gfo_transpose_last2(const float *in, float *out, size_t batch,
                                 size_t rows, size_t cols) {
    for (size_t bi = 0; bi < batch; ++bi) {
        const float *s = in + bi * rows * cols;
        float *d = out + bi * rows * cols;
        for (size_t j = 0; j < cols; ++j)
            for (size_t i = 0; i < rows; ++i)
                d[j * rows + i] = s[i * cols + j];
    }
}

/* ------------------------------------------------------------------------ */
/* ghostflow-core/src/ops/arithmetic.rs                                      */
/* ------------------------------------------------------------------------ */

/* arithmetic.rs:20-27 + :124-215: `[rows, cols] + [cols]` takes the broadcast
 * path; the bias index is the flat index with the row coordinate's stride 0,
 * i.e. out[i] = y[i] + b[i % cols], one rounding. */
GFO_API void gfo_add_row_bias(float *y, const float *bias, size_t rows,
                              size_t cols) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) y[r * cols + c] = y[r * cols + c] + bias[c];
}

/* arithmetic.rs:69-72 `mul_scalar`: x * s. */
GFO_API void gfo_mul_scalar(float *x, size_t n, float s) {
    for (size_t i = 0; i < n; ++i) x[i] = x[i] * s;
}

/* ------------------------------------------------------------------------ */
/* ghostflow-autograd/src/backward.rs                                        */
/* ------------------------------------------------------------------------ */

/* backward.rs:131-160 `matmul_backward`: grad [m,n], a [m,k], b [k,n];
 * grad_a[i,j] = sum_l grad[i,l] * b[j,l]  (grad . b^T, l ascending),
 * grad_b[i,j] = sum_l a[l,i] * grad[l,j]  (a^T . grad, l ascending);
 * each sum starts from 0.0f and adds separately rounded products.  Either
 * output may be NULL. */
GFO_API void gfo_matmul_backward(const float *grad, const float *a, const float *b,
                                 size_t m, size_t k, size_t n, float *grad_a,
                                 float *grad_b) {
    if (grad_a)
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < k; ++j) {
                float sum = 0.0f;
                for (size_t l = 0; l < n; ++l) sum = sum + grad[i * n + l] * b[j * n + l];
                grad_a[i * k + j] = sum;
            }
    if (grad_b)
        for (size_t i = 0; i < k; ++i)
            for (size_t j = 0; j < n; ++j) {
                float sum = 0.0f;
                for (size_t l = 0; l < m; ++l) sum = sum + a[l * k + i] * grad[l * n + j];
                grad_b[i * n + j] = sum;
            }
}

/* ------------------------------------------------------------------------ */
/* ghostflow-nn/src/linear.rs                                                */
/* ------------------------------------------------------------------------ */

/* linear.rs:56-69 `Linear::forward`: weight.t() (view), materialized by
 * data_f32 inside matmul_blocked, then `output.add(bias)`. */
GFO_API int gfo_linear_forward(const float *x, const float *w, const float *bias,
                               float *y, size_t m, size_t in_f, size_t out_f) {
    float *wt = (float *)malloc(in_f * out_f * sizeof(float) + 1);
    if (!wt) return 4;
    gfo_transpose_last2(w, wt, 1, out_f, in_f); /* [out,in] -> [in,out] */
    gfo_matmul_blocked(x, wt, y, m, in_f, out_f);
    free(wt);
    if (bias) gfo_add_row_bias(y, bias, m, out_f);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* ghostflow-core/src/ops/activation.rs                                      */
/* ------------------------------------------------------------------------ */

/* activation.rs:165-216 `softmax(-1)` (inner_size == 1): per row,
 * max = fold(-inf, f32::max) (NaN-ignoring, = fmaxf); e_j = expf(x_j - max)
 * with `sum += e_j` ascending; then e_j / sum (true division).  f32::exp is
 * llvm.exp.f32, which lowers to the platform libm expf. */
GFO_API void gfo_softmax_lastdim(const float *x, float *y, size_t rows,
                                 size_t cols) {
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * cols;
        float *yr = y + r * cols;
        float mx = -INFINITY;
        for (size_t j = 0; j < cols; ++j) mx = fmaxf(mx, xr[j]);
        float sum = 0.0f;
        for (size_t j = 0; j < cols; ++j) {
            float e = expf(xr[j] - mx);
            yr[j] = e;
            sum = sum + e;
        }
        for (size_t j = 0; j < cols; ++j) yr[j] = yr[j] / sum;
    }
}

/* activation.rs:117-122 `silu` = x / (1.0 + (-x).exp()) (negate, expf, add,
 * true division: three roundings), then arithmetic.rs:39-45 `mul` of two
 * same-shaped tensors (one rounding): the `gate.silu().mul(&up)` step of
 * SwiGLU::forward (ghostflow-nn/src/llama.rs:276-286). */
GFO_API void gfo_silu_mul(const float *gate, const float *up, float *out,
                          size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float g = gate[i];
        const float s = g / (1.0f + expf(-g));
        out[i] = s * up[i];
    }
}

/* ------------------------------------------------------------------------ */
/* ghostflow-nn/src/attention.rs, ghostflow-cuda/src/ops.rs                  */
/* ------------------------------------------------------------------------ */

/* attention.rs:51-64 `apply_attention_mask`: the flattened mask is CYCLED
 * over all scores; m > 0.5 keeps the score, otherwise -inf. */
GFO_API void gfo_apply_mask_cycled(float *scores, size_t n, const float *mask,
                                   size_t mask_n) {
    for (size_t i = 0; i < n; ++i)
        if (!(mask[i % mask_n] > 0.5f)) scores[i] = -INFINITY;
}

/* ghostflow-cuda/src/ops.rs:205-224 `apply_causal_mask`: j > i -> -inf in
 * every [S,S] slice. */
GFO_API void gfo_apply_causal(float *scores, size_t batch, size_t s) {
    for (size_t bi = 0; bi < batch; ++bi)
        for (size_t i = 0; i < s; ++i)
            for (size_t j = i + 1; j < s; ++j) scores[bi * s * s + i * s + j] = -INFINITY;
}

/* Shared body of attention.rs:11-49 and ops.rs:166-203:
 *   scores = Q.matmul(K^T)      (batched_matmul, K^T materialized)
 *   scores = scores * scale     (mul_scalar: rounded AFTER the k-sum)
 *   mask                        (cycled mask or causal)
 *   w      = softmax(-1)
 *   out    = w.matmul(V)
 * Q [bh, sq, d], K/V [bh, skv, d].  `weights` (nullable) receives w. */
static int sdpa_body(const float *q, const float *k, const float *v, float *out,
                     float *weights, size_t bh, size_t sq, size_t skv, size_t d,
                     float scale, const float *mask, size_t mask_n, int causal) {
    float *kt = (float *)malloc(bh * skv * d * sizeof(float) + 1);
    float *sc = (float *)malloc(bh * sq * skv * sizeof(float) + 1);
    float *w = weights ? weights : (float *)malloc(bh * sq * skv * sizeof(float) + 1);
    if (!kt || !sc || !w) {
        free(kt); free(sc); if (!weights) free(w);
        return 4;
    }
    gfo_transpose_last2(k, kt, bh, skv, d);
    gfo_batched_matmul(q, bh, kt, bh, sc, bh, sq, d, skv);
    gfo_mul_scalar(sc, bh * sq * skv, scale);
    if (mask) gfo_apply_mask_cycled(sc, bh * sq * skv, mask, mask_n);
    if (causal) gfo_apply_causal(sc, bh, sq); /* ops.rs assumes sq == skv */
    gfo_softmax_lastdim(sc, w, bh * sq, skv);
    gfo_batched_matmul(w, bh, v, bh, out, bh, sq, skv, d);
    free(kt); free(sc);
    if (!weights) free(w);
    return 0;
}

/* attention.rs:11-49 `scaled_dot_product_attention` (dropout off: the
 * inference path, :37-43).  scale = 1.0 / (d as f32).sqrt() (:19-20). */
GFO_API int gfo_sdpa(const float *q, const float *k, const float *v,
                     const float *mask, size_t mask_n, float *out, float *weights,
                     size_t bh, size_t sq, size_t skv, size_t d) {
    float scale = 1.0f / sqrtf((float)d);
    return sdpa_body(q, k, v, out, weights, bh, sq, skv, d, scale, mask, mask_n, 0);
}

/* ghostflow-cuda/src/ops.rs:166-203 `flash_attention(q,k,v,scale,causal)`:
 * the GPU-API entry of the same computation with the scale passed in and the
 * causal mask of :205-224. */
GFO_API int gfo_flash_attention(const float *q, const float *k, const float *v,
                                float *out, size_t bh, size_t s, size_t d,
                                float scale, int causal) {
    return sdpa_body(q, k, v, out, NULL, bh, s, s, d, scale, NULL, 0, causal);
}

/* Rows [r0, r1) of one (b,h) slice of the flash path (rows are
 * independent: each needs Q row i and all of K, V), for checks of sampled
 * rows of a large slice. */
GFO_API int gfo_flash_attention_rows(const float *q, const float *k, const float *v,
                                     float *out, size_t s, size_t d, float scale,
                                     int causal, size_t r0, size_t r1) {
    size_t rows = r1 - r0;
    float *kt = (float *)malloc(s * d * sizeof(float) + 1);
    float *sc = (float *)malloc(rows * s * sizeof(float) + 1);
    float *w = (float *)malloc(rows * s * sizeof(float) + 1);
    if (!kt || !sc || !w) { free(kt); free(sc); free(w); return 4; }
    gfo_transpose_last2(k, kt, 1, s, d);
    gfo_batched_matmul(q + r0 * d, 1, kt, 1, sc, 1, rows, d, s);
    gfo_mul_scalar(sc, rows * s, scale);
    if (causal)
        for (size_t i = 0; i < rows; ++i)
            for (size_t j = r0 + i + 1; j < s; ++j) sc[i * s + j] = -INFINITY;
    gfo_softmax_lastdim(sc, w, rows, s);
    gfo_batched_matmul(w, 1, v, 1, out + r0 * d, 1, rows, s, d);
    free(kt); free(sc); free(w);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* ghostflow-nn/src/flash_attention.rs                                       */
/* ------------------------------------------------------------------------ */

/* flash_attention.rs:81-250 `FlashAttention::forward` on [batch, sq, d] query
 * and [batch, sk, d] key / value, each batch independently (:106-116,
 * extract_batch :253-264, concatenate_batches :266-282):
 *   output = 0, row_max = -inf, row_sum = 0                       (:135-137)
 *   for query blocks i0 (block_m), key blocks j0 (block_n)        (:143-163)
 *     skip when causal && j0 >= end_i                             (:150-152)
 *     process_block (:178-250), per row i of the query block:
 *       score_j = (sum_d q*k, ascending, from 0.0) * scale, or -inf when
 *                 causal && j > i (absolute indices: top-left)    (:193-206)
 *       block_max = fold(-inf, f32::max) over unmasked scores     (:208)
 *       new_max = max(old_max, block_max)                         (:212-214)
 *       p_j = exp(score_j - new_max), 0 for masked; block_sum += p_j  (:217-226)
 *       correction = exp(old_max - new_max)                       (:229)
 *       row_sum = row_sum * correction + block_sum                (:230)
 *       for every key j of the block (masked ones included):
 *         output = output * correction + p_j * v_j                (:233-241)
 *   output /= row_sum where row_sum > 0                           (:166-172)
 * The correction multiplies the output once PER KEY of the block (:236-237),
 * not once per block: the first block (correction = exp(-inf) = 0) keeps
 * only its last key, and a later block whose max rises scales the earlier
 * output by correction^(keys in the block).  With block_n == 1 this is the
 * exact online softmax.  Returns 1 for a zero block size (Rust's step_by(0)
 * panics), 4 on allocation failure. */
GFO_API int gfo_flash_attention_blockwise(const float *q, const float *k, const float *v,
                                          float *out, size_t batch, size_t sq, size_t sk,
                                          size_t d, size_t block_m, size_t block_n,
                                          int causal, float scale) {
    if (block_m == 0 || block_n == 0) return 1;
    float *row_max = (float *)malloc(sq * sizeof(float) + 1);
    float *row_sum = (float *)malloc(sq * sizeof(float) + 1);
    float *scores = (float *)malloc(block_n * sizeof(float) + 1);
    if (!row_max || !row_sum || !scores) {
        free(row_max); free(row_sum); free(scores);
        return 4;
    }
    for (size_t b = 0; b < batch; ++b) {
        const float *qb = q + b * sq * d, *kb = k + b * sk * d, *vb = v + b * sk * d;
        float *ob = out + b * sq * d;
        for (size_t i = 0; i < sq * d; ++i) ob[i] = 0.0f;
        for (size_t i = 0; i < sq; ++i) {
            row_max[i] = -INFINITY;
            row_sum[i] = 0.0f;
        }
        for (size_t i0 = 0; i0 < sq; i0 += block_m) {
            const size_t end_i = i0 + block_m < sq ? i0 + block_m : sq;
            for (size_t j0 = 0; j0 < sk; j0 += block_n) {
                const size_t end_j = j0 + block_n < sk ? j0 + block_n : sk;
                if (causal && j0 >= end_i) continue;
                for (size_t i = i0; i < end_i; ++i) {
                    float block_max = -INFINITY;
                    size_t ns = 0;
                    for (size_t j = j0; j < end_j; ++j) {
                        if (causal && j > i) {
                            scores[ns++] = -INFINITY;
                            continue;
                        }
                        float score = 0.0f;
                        for (size_t t = 0; t < d; ++t) {
                            float p = qb[i * d + t] * kb[j * d + t];
                            score = score + p;
                        }
                        score = score * scale;
                        scores[ns++] = score;
                        block_max = fmaxf(block_max, score);
                    }
                    const float old_max = row_max[i];
                    const float new_max = fmaxf(old_max, block_max);
                    row_max[i] = new_max;
                    float block_sum = 0.0f;
                    for (size_t t = 0; t < ns; ++t) {
                        if (scores[t] != -INFINITY) {
                            scores[t] = expf(scores[t] - new_max);
                            block_sum = block_sum + scores[t];
                        } else {
                            scores[t] = 0.0f;
                        }
                    }
                    const float correction = expf(old_max - new_max);
                    {
                        float t1 = row_sum[i] * correction;
                        row_sum[i] = t1 + block_sum;
                    }
                    for (size_t t = 0; t < ns; ++t) {
                        const size_t j = j0 + t;
                        if (j < sk)
                            for (size_t e = 0; e < d; ++e) {
                                float t1 = ob[i * d + e] * correction;
                                float t2 = scores[t] * vb[j * d + e];
                                ob[i * d + e] = t1 + t2;
                            }
                    }
                }
            }
        }
        for (size_t i = 0; i < sq; ++i)
            if (row_sum[i] > 0.0f)
                for (size_t e = 0; e < d; ++e) ob[i * d + e] = ob[i * d + e] / row_sum[i];
    }
    free(row_max); free(row_sum); free(scores);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* ghostflow-nn/src/quantization.rs                                          */
/* ------------------------------------------------------------------------ */

/* The (scale, zero_point) pair of one group, quantization.rs:78-91
 * (per tensor) and :124-135 (per channel):
 *   min = fold(+inf, f32::min), max = fold(-inf, f32::max)  (NaN-ignoring)
 *   symmetric : scale = max(|min|, |max|) / 127, zp = 0
 *   asymmetric: scale = (max - min) / 255,
 *               zp = ((-min / scale) - 128.0).round() as i8   (saturating) */
static void quant_params(const float *x, size_t n, int symmetric, float *scale_out,
                         int8_t *zp_out) {
    float mn = INFINITY, mx = -INFINITY;
    for (size_t i = 0; i < n; ++i) mn = fminf(mn, x[i]);
    for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, x[i]);
    if (symmetric) {
        float absmax = fmaxf(fabsf(mn), fabsf(mx));
        *scale_out = absmax / 127.0f;
        *zp_out = 0;
    } else {
        float scale = (mx - mn) / 255.0f;
        float t = (-mn) / scale;
        t = t - 128.0f;
        *scale_out = scale;
        *zp_out = rust_f32_as_i8(roundf(t));
    }
}

/* quantization.rs:96-97 / :141-142:
 *   q = ((x / scale).round() as i32 + zp as i32).clamp(-128, 127) as i8
 * `round` is half away from zero (C roundf); `as i32` saturates, NaN -> 0. */
static int8_t quant_one(float x, float scale, int8_t zp) {
    int32_t q = rust_wrapping_add_i32(rust_f32_as_i32(roundf(x / scale)), (int32_t)zp);
    if (q < -128) q = -128;
    if (q > 127) q = 127;
    return (int8_t)q;
}

/* quantization.rs:77-108 `quantize_per_tensor_int8`. */
GFO_API void gfo_quantize_per_tensor(const float *x, size_t n, int symmetric,
                                     int8_t *q, float *scale, int8_t *zp) {
    quant_params(x, n, symmetric, scale, zp);
    for (size_t i = 0; i < n; ++i) q[i] = quant_one(x[i], *scale, *zp);
}

/* quantization.rs:110-153 `quantize_per_channel_int8`: channel = dim 0,
 * each channel a contiguous run of numel/shape[0] elements. */
GFO_API void gfo_quantize_per_channel(const float *x, size_t rows, size_t cols,
                                      int symmetric, int8_t *q, float *scales,
                                      int8_t *zps) {
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * cols;
        quant_params(xr, cols, symmetric, &scales[r], &zps[r]);
        for (size_t c = 0; c < cols; ++c) q[r * cols + c] = quant_one(xr[c], scales[r], zps[r]);
    }
}

/* quantization.rs:173-204 `dequantize_int8`: one scale -> per tensor,
 * otherwise per channel over dim 0; value = (q as f32 - zp as f32) * scale. */
GFO_API void gfo_dequantize(const int8_t *q, size_t rows, size_t cols,
                            const float *scales, const int8_t *zps, size_t nscales,
                            float *out) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) {
            size_t g = nscales == 1 ? 0 : r;
            float d = (float)q[r * cols + c] - (float)zps[g];
            out[r * cols + c] = d * scales[g];
        }
}

/* ------------------------------------------------------------------------ */
/* INT8 linear (defined on top of the reference scheme; the reference has no  */
/* integer GEMM -- its executable path is dequantize + fp32 matmul,          */
/* quantization.rs:275-277)                                                   */
/* ------------------------------------------------------------------------ */

/* acc[m,n] = sum_k (qx[m,k] - zx[m']) * qw[n,k]   (exact int32)
 * x_per_row == 0 : one (sx, zx) for all of x  (DynamicQuantization::
 *                  quantize_activation, quantization.rs:280-287)
 * x_per_row == 1 : (sx[m], zx[m]) per row      (QuantizationConfig::default,
 *                  per-channel over dim 0 of x)
 * y[m,n] = ((float)acc * (sx * sw[n])) + b[n]  -- sx*sw rounded once, then
 * the product, then the bias add; each a separate f32 rounding. */
GFO_API void gfo_qlinear_i8(const int8_t *qx, const float *sx, const int8_t *zx,
                            int x_per_row, const int8_t *qw, const float *sw,
                            const float *bias, float *y, int32_t *acc_out,
                            size_t m, size_t n, size_t k) {
    for (size_t i = 0; i < m; ++i) {
        size_t g = x_per_row ? i : 0;
        int32_t z = zx ? (int32_t)zx[g] : 0;
        for (size_t j = 0; j < n; ++j) {
            int64_t acc = 0;
            for (size_t kk = 0; kk < k; ++kk)
                acc += (int64_t)((int32_t)qx[i * k + kk] - z) * (int64_t)qw[j * k + kk];
            int32_t a32 = (int32_t)acc;
            if (acc_out) acc_out[i * n + j] = a32;
            if (y) {
                float s = sx[g] * sw[j];
                float v = (float)a32 * s;
                if (bias) v = v + bias[j];
                y[i * n + j] = v;
            }
        }
    }
}
