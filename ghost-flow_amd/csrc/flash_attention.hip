// flash_attention.hip -- FlashAttention::forward
// (ghostflow-nn/src/flash_attention.rs:81-250) on q [batch, sq, d], k / v
// [batch, sk, d] with FlashAttentionConfig's block sizes, causal flag and
// scale.
//
// The reference walks query blocks (block_m) and key blocks (block_n) with a
// running row max m, row sum l and output o.  Per row and processed key block
// t (n_t keys, running max m_t after it, delta_t = m_{t-1} - m_t <= 0):
//   p_j = exp(s_j - m_t) (0 for a masked key), c_t = exp(delta_t),
//   l   = l * c_t + sum_j p_j,
//   and for EVERY key of the block, masked ones included (:233-241):
//   o   = o * c_t + p_j * v_j,
// i.e. the correction multiplies the output once per key, not once per
// block.  Unrolled, the output is a fixed linear combination of the rows of
// v:
//   o = sum_t sum_{j in t} p_j c_t^(n_t - 1 - idx_j) prod_{t' > t} c_t'^n_t' v_j
// where the first block has c_0 = exp(-inf) = 0 (only its last key survives),
// and l = sum_j exp(s_j - m_last).  So the layer runs as
//   1. S = scale * Q . K^T                 (gfh_sgemm NT, alpha = scale: the
//                                            scale rounds the finished sum,
//                                            `score *= scale`, :203)
//   2. S -> W in place, one workgroup per row: block maxima, their running
//      max (a scan), the suffix sums of n_t' delta_t' (a scan), l, then
//      W_j = exp(s_j - m_t + (n_t - 1 - idx) delta_t + sum_{t'>t} n_t'
//      delta_t') / l, with the log-weights summed before one exp;
//   3. O = W . V                             (gfh_sgemm NN).
// Causal masking uses absolute indices, key j visible to row i iff j <= i
// (top-left, :193-196), and key blocks starting at or past the end of the
// row's query block are skipped (:150-152).  The result is the reference's
// within fp32 rounding (different summation orders, and c^e evaluated as
// exp(e delta)); non-finite inputs are outside that contract.  With
// block_n = 1 the recurrence is exact softmax attention.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

// Every f32 product and sum is its own rounding, as in the reference CPU
// path (no FMA contraction).
#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kFaThreads = 256;

struct FaRow {
    float *w;  // [rows][sk] scores in, weights out
    int64_t sq, sk, bm, bn;
    int causal;
};

// Inclusive scan of one float per thread over the workgroup with `op`
// (Hillis-Steele through LDS); every thread gets its own prefix.
template <typename Op>
__device__ __forceinline__ float wg_inclusive_scan(float v, float *buf, Op op) {
    const int tid = threadIdx.x;
    buf[tid] = v;
    __syncthreads();
#pragma unroll
    for (int off = 1; off < kFaThreads; off <<= 1) {
        const float o = tid >= off ? buf[tid - off] : v;
        __syncthreads();
        if (tid >= off) v = op(v, o);
        buf[tid] = v;
        __syncthreads();
    }
    return v;
}

// NB: LDS capacity for per-block state (block maxima, suffix sums).
template <int NB>
__global__ __launch_bounds__(kFaThreads) void fa_weights_kernel(FaRow p) {
    __shared__ float M[NB];  // block max, then the running max after each block
    __shared__ float E[NB];  // sum over later processed blocks of n * delta
    __shared__ float buf[kFaThreads];
    __shared__ float red[kFaThreads / 64];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t i = row % p.sq;
    float *s = p.w + row * p.sk;
    const int64_t nb = (p.sk + p.bn - 1) / p.bn;
    // Processed key blocks: all, or (causal) those starting before the end
    // of this row's query block.  Visible keys: j < jv.
    const int64_t end_i = std::min<int64_t>((i / p.bm + 1) * p.bm, p.sq);
    const int64_t np = p.causal ? std::min<int64_t>(nb, (end_i + p.bn - 1) / p.bn) : nb;
    const int64_t jv = p.causal ? std::min<int64_t>(p.sk, i + 1) : p.sk;

    // 1. block maxima over the visible keys (-inf for a block with none)
    for (int64_t t = tid; t < np; t += kFaThreads) {
        const int64_t j0 = t * p.bn, j1 = std::min<int64_t>(std::min<int64_t>(j0 + p.bn, p.sk), jv);
        float mx = -INFINITY;
        for (int64_t j = j0; j < j1; ++j) mx = fmaxf(mx, s[j]);
        M[t] = mx;
    }
    __syncthreads();

    // 2. running max: each thread folds a chunk of consecutive blocks, the
    // chunk maxima are scanned across the workgroup, then the chunk is
    // rewritten with the prefix from the chunks before it.
    const int64_t chunk = (np + kFaThreads - 1) / kFaThreads;
    const int64_t lo = std::min<int64_t>(tid * chunk, np), hi = std::min<int64_t>(lo + chunk, np);
    float run = -INFINITY;
    for (int64_t t = lo; t < hi; ++t) run = fmaxf(run, M[t]);
    const float incl = wg_inclusive_scan(run, buf, [](float a, float b) { return fmaxf(a, b); });
    float before = tid > 0 ? buf[tid - 1] : -INFINITY;
    (void)incl;
    __syncthreads();
    for (int64_t t = lo; t < hi; ++t) {
        before = fmaxf(before, M[t]);
        M[t] = before;
    }
    __syncthreads();

    // 3. E[t] = sum over processed t' > t of n_t' (M[t'-1] - M[t']): the
    // chunk sums scanned from the back (suffix), then each chunk walked
    // backwards.
    auto term = [&](int64_t t) -> float {
        const float n = (float)std::min<int64_t>(p.bn, p.sk - t * p.bn);
        return n * (M[t - 1] - M[t]);
    };
    float part = 0.f;
    for (int64_t t = std::max<int64_t>(lo, 1); t < hi; ++t) part = part + term(t);
    // suffix scan = prefix scan over reversed thread order
    buf[kFaThreads - 1 - tid] = part;
    __syncthreads();
    const float mine = buf[tid];
    __syncthreads();
    const float rincl = wg_inclusive_scan(mine, buf, [](float a, float b) { return a + b; });
    (void)rincl;
    // exclusive suffix of thread tid = inclusive prefix of reversed index (255 - tid) - 1
    const int rt = kFaThreads - 1 - tid;
    float after = rt > 0 ? buf[rt - 1] : 0.f;
    __syncthreads();
    for (int64_t t = hi - 1; t >= lo; --t) {
        E[t] = after;
        if (t >= 1) after = after + term(t);
    }
    __syncthreads();

    // 4. l = sum of exp(s_j - m_last) over the visible keys
    const float m_last = np > 0 ? M[np - 1] : -INFINITY;
    float ls = 0.f;
    for (int64_t j = tid; j < jv; j += kFaThreads) ls = ls + expf(s[j] - m_last);
    ls = wave_sum(ls);
    if ((tid & 63) == 0) red[tid >> 6] = ls;
    __syncthreads();
    const float l = (red[0] + red[1]) + (red[2] + red[3]);

    // 5. the weights, in place (each thread rewrites only the keys it read
    // in step 4's loop order)
    for (int64_t j = tid; j < p.sk; j += kFaThreads) {
        float out = 0.f;
        if (j < jv) {
            const int64_t t = j / p.bn, idx = j - t * p.bn;
            const int64_t n = std::min<int64_t>(p.bn, p.sk - t * p.bn);
            float lw;
            if (t == 0)
                lw = idx == n - 1 ? (s[j] - M[0]) + E[0] : -INFINITY;
            else
                lw = ((s[j] - M[t]) + (float)(n - 1 - idx) * (M[t - 1] - M[t])) + E[t];
            const float e = expf(lw);
            out = l > 0.f ? e / l : e;
        }
        s[j] = out;
    }
}

__global__ void fa_zero_kernel(float *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.f;
}

}  // namespace

int64_t flash_attention_max_blocks() { return 8192; }

int launch_flash_attention_blockwise(const FlashAttnDesc &d, hipStream_t s) {
    if (d.batch == 0 || d.sq == 0 || d.d == 0) return GFH_SUCCESS;
    const bool big_batch = d.batch > 16;
    // 1. S = scale * Q . K^T  (per batch element when the single-GEMM tile
    //    kernels fit, else one strided-batched call)
    auto gemm = [&](bool nt, const float *a, int64_t lda, int64_t sa, const float *b, int64_t ldb, int64_t sb,
                    float *c, int64_t ldc, int64_t sc, int64_t m, int64_t n, int64_t k, float alpha) -> int {
        SgemmDesc g;
        g.trans_b = nt;
        g.m = m;
        g.n = n;
        g.k = k;
        g.alpha = alpha;
        g.a = a;
        g.lda = lda;
        g.b = b;
        g.ldb = ldb;
        g.c = c;
        g.ldc = ldc;
        if (!big_batch && sa % 4 == 0 && sb % 4 == 0 && sc % 4 == 0 && sgemm_big_fits(g)) {
            for (int64_t bi = 0; bi < d.batch; ++bi) {
                g.a = a + bi * sa;
                g.b = b + bi * sb;
                g.c = c + bi * sc;
                GFH_TRY(launch_sgemm(g, s));
            }
            return GFH_SUCCESS;
        }
        g.stride_a = sa;
        g.stride_b = sb;
        g.stride_c = sc;
        g.batch_a = d.batch;
        g.batch_b = d.batch;
        g.batch = d.batch;
        return launch_sgemm(g, s);
    };
    if (d.sk == 0) {  // no keys: the reference's output stays 0 (row_sum 0, no division)
        const int64_t n = d.batch * d.sq * d.d;
        hipLaunchKernelGGL(fa_zero_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)), dim3(256), 0,
                           s, d.out, n);
        return check_launch("flash_attention (zero output)");
    }
    {
        GFH_TRY(gemm(true, d.q, d.d, d.sq * d.d, d.k, d.d, d.sk * d.d, d.ws, d.sk, d.sq * d.sk, d.sq, d.sk, d.d,
                     d.scale));
        // 2. blockwise weights, in place
        FaRow r;
        r.w = d.ws;
        r.sq = d.sq;
        r.sk = d.sk;
        r.bm = d.block_m;
        r.bn = d.block_n;
        r.causal = d.causal ? 1 : 0;
        const int64_t nb = (d.sk + d.block_n - 1) / d.block_n;
        const dim3 grid((unsigned)(d.batch * d.sq)), block(kFaThreads);
        if (nb <= 256)
            hipLaunchKernelGGL(fa_weights_kernel<256>, grid, block, 0, s, r);
        else
            hipLaunchKernelGGL(fa_weights_kernel<8192>, grid, block, 0, s, r);
        GFH_TRY(check_launch("flash_attention (weights)"));
    }
    // 3. O = W . V
    return gemm(false, d.ws, d.sk, d.sq * d.sk, d.v, d.d, d.sk * d.d, d.out, d.d, d.sq * d.d, d.sq, d.d, d.sk,
                1.0f);
}

}  // namespace gfh
