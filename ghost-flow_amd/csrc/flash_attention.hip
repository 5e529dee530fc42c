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
// and l = sum_j exp(s_j - m_last).  Three forms compute it:
//   * fa_onepass_kernel (block_n = 32 or 64): the recurrence per key block
//     in closed form, one pass (below);
//   * fa_fused_kernel (other multiples of 32): two passes, the block maxima
//     first (below);
//   * otherwise three steps:
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
// row's query block are skipped (:150-152).  The block maxima M_t are
// exact (fp64 scores of their keys, kept in fp64: see exact_dot), so the
// result differs from the exact value of the recurrence only by the
// rounding of each key's own fp32 score and weight -- closer to it than the
// reference's own fp32 evaluation, whose max errors the recurrence amplifies
// -- and from the reference by that amount (different summation orders, c^e
// evaluated as exp(e delta)); non-finite inputs are outside that contract.
// With block_n = 1 the recurrence is exact softmax attention.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "attn_tiles.hpp"
#include "common.hpp"
#include "kernels.hpp"

// Every f32 product and sum is its own rounding, as in the reference CPU
// path (no FMA contraction).
#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kFaThreads = 256;

struct FaRow {
    float *w;            // [rows][sk] scores in, weights out
    const float *q, *k;  // [batch][sq][d], [batch][sk][d]: exact block maxima
    int64_t sq, sk, d, bm, bn;
    float scale;
    int causal;
};

// Inclusive scan of one value per thread over the workgroup with `op`
// (Hillis-Steele through LDS); every thread gets its own prefix.
template <typename T, typename Op>
__device__ __forceinline__ T wg_inclusive_scan(T v, T *buf, Op op) {
    const int tid = threadIdx.x;
    buf[tid] = v;
    __syncthreads();
#pragma unroll
    for (int off = 1; off < kFaThreads; off <<= 1) {
        const T o = tid >= off ? buf[tid - off] : v;
        __syncthreads();
        if (tid >= off) v = op(v, o);
        buf[tid] = v;
        __syncthreads();
    }
    return v;
}

// NB: LDS capacity for per-block state (block maxima, suffix sums), kept in
// fp64: each block's maximum is the exact score of its key with the largest
// fp32 score (q . k summed in fp64, times the scale), for the reason given
// with tile_argmax / exact_dot below.
template <int NB>
__global__ __launch_bounds__(kFaThreads) void fa_weights_kernel(FaRow p) {
    __shared__ double M[NB];  // block max, then the running max after each block
    __shared__ double E[NB];  // sum over later processed blocks of n * delta
    __shared__ double buf[kFaThreads];
    __shared__ float red[kFaThreads / 64];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t i = row % p.sq;
    float *s = p.w + row * p.sk;
    const float *qrow = p.q + row * p.d;
    const float *kb = p.k + (row / p.sq) * p.sk * p.d;
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
        int64_t jm = -1;
        for (int64_t j = j0; j < j1; ++j)
            if (s[j] > mx) {
                mx = s[j];
                jm = j;
            }
        double ex = -INFINITY;
        if (jm >= 0) {
            const float *krow = kb + jm * p.d;
            double dot = 0.0;
            for (int64_t e = 0; e < p.d; ++e) dot = fma((double)qrow[e], (double)krow[e], dot);
            ex = dot * (double)p.scale;
        }
        M[t] = ex;
    }
    __syncthreads();

    // 2. running max: each thread folds a chunk of consecutive blocks, the
    // chunk maxima are scanned across the workgroup, then the chunk is
    // rewritten with the prefix from the chunks before it.
    const int64_t chunk = (np + kFaThreads - 1) / kFaThreads;
    const int64_t lo = std::min<int64_t>(tid * chunk, np), hi = std::min<int64_t>(lo + chunk, np);
    double run = -INFINITY;
    for (int64_t t = lo; t < hi; ++t) run = fmax(run, M[t]);
    (void)wg_inclusive_scan(run, buf, [](double a, double b) { return fmax(a, b); });
    double before = tid > 0 ? buf[tid - 1] : -INFINITY;
    __syncthreads();
    for (int64_t t = lo; t < hi; ++t) {
        before = fmax(before, M[t]);
        M[t] = before;
    }
    __syncthreads();

    // 3. E[t] = sum over processed t' > t of n_t' (M[t'-1] - M[t']): the
    // chunk sums scanned from the back (suffix), then each chunk walked
    // backwards.
    auto term = [&](int64_t t) -> double {
        const double n = (double)std::min<int64_t>(p.bn, p.sk - t * p.bn);
        return n * (M[t - 1] - M[t]);
    };
    double part = 0.0;
    for (int64_t t = std::max<int64_t>(lo, 1); t < hi; ++t) part = part + term(t);
    // suffix scan = prefix scan over reversed thread order
    buf[kFaThreads - 1 - tid] = part;
    __syncthreads();
    const double mine = buf[tid];
    __syncthreads();
    (void)wg_inclusive_scan(mine, buf, [](double a, double b) { return a + b; });
    // exclusive suffix of thread tid = inclusive prefix of reversed index (255 - tid) - 1
    const int rt = kFaThreads - 1 - tid;
    double after = rt > 0 ? buf[rt - 1] : 0.0;
    __syncthreads();
    for (int64_t t = hi - 1; t >= lo; --t) {
        E[t] = after;
        if (t >= 1) after = after + term(t);
    }
    __syncthreads();

    // 4. l = sum of exp(s_j - m_last) over the visible keys
    const float m_last = np > 0 ? (float)M[np - 1] : -INFINITY;
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
                lw = idx == n - 1 ? (s[j] - (float)M[0]) + (float)E[0] : -INFINITY;
            else
                lw = ((s[j] - (float)M[t]) + (float)(n - 1 - idx) * (float)(M[t - 1] - M[t])) + (float)E[t];
            const float e = expf(lw);
            out = l > 0.f ? e / l : e;
        }
        s[j] = out;
    }
}

// ---- fused two-pass form --------------------------------------------------
//
// With block_n a multiple of the 32-key tile, each tile lies in one key
// block and the weights need, per row, only the running max M_t after each
// block: for t >= 1
//   W_j = exp((s_j - M_t) + (n_t - 1 - idx_j) (M_{t-1} - M_t) + E_t) / l,
// block 0 keeping only its last key, and E_t = sum over later blocks t' <= V
// of n_t' (M_{t'-1} - M_t') -- V the last block holding a visible key (later
// processed blocks are fully masked: M stays, they add nothing).  Every block
// before V is full (n = block_n), so the sum telescopes:
//   E_t = block_n (M_t - M_{V-1}) + n_V (M_{V-1} - M_V),  E_V = 0.
// One workgroup per 128 queries (4 waves x 32) of one batch element, laid
// out as the SDPA kernel (S^T = K . Q^T on v_mfma_f32_32x32x2_f32, lane =
// query, 32-key K / V tiles double-buffered through LDS):
//   pass 1: scores tile by tile; the online max m and sum l (l = sum of
//           exp(s_j - M_V) over the visible keys); m after a block's last
//           tile is M_t, written to mblk[row][t];
//   pass 2: the same scores again (same instructions, so the same bits),
//           W_j (unnormalized) from mblk, and O += W . V on the MFMA with the
//           weights straight from the score registers; O / l at the end.
// Work: 1.5x the matmul FLOPs of plain attention, no score matrix in HBM.
// Keys are processed up to the workgroup's last query (causal) or all of
// them: the reference's skip of blocks past a query block (:150-152) only
// skips fully masked blocks, which change neither M nor O.
struct FaFused {
    const float *q, *k, *v;
    float *out;
    double *mblk;  // [batch * sq][nbw] exact running maxima
    int64_t sq, sk, d, bn, nbw;
    float scale;
    int nqb, fold;
};

constexpr int kFaBQ = 128;  // queries per workgroup

// ---- exact block maxima ---------------------------------------------------------
//
// The recurrence multiplies the output by exp(M_{t-1} - M_t) once per key, so
// an error in a running max M enters the exponent up to block_n times (and
// the later blocks' sizes times more).  An fp32 score of a length-d dot
// product is off from the exact one by ~1e-6 of its size (the reference's
// own fp32 evaluation suffers the same), enough for relative errors of
// ~1e-5 after that amplification.  So every block maximum is recomputed
// exactly: the key with the largest fp32 score has q . k summed in fp64
// (a product of two fp32 values is exact in fp64), times the fp32 scale,
// and the running maxima and their differences are kept in fp64.  The
// weights then carry only the unamplified rounding of each key's own score.

// This row's largest fp32 score of a 32-key tile, and its key: lanes (c, 0)
// and (c, 1) hold keys key_of(r, 0) / key_of(r, 1) and both get the same
// answer (ties go to lane half 0, then to the lower register).  A row with
// no visible key gets -inf and key 0.
__device__ __forceinline__ int tile_argmax(const float (&x)[16], int h, float &mx) {
    float m = x[0];
    int rb = 0;
#pragma unroll
    for (int r = 1; r < 16; ++r)
        if (x[r] > m) {
            m = x[r];
            rb = r;
        }
    const int kb = m == -INFINITY ? 0 : attn::key_of(rb, h);
    const float pm = __shfl_xor(m, 32);
    const int pk = __shfl_xor(kb, 32);
    const float m0 = h ? pm : m, m1 = h ? m : pm;
    const int k0 = h ? pk : kb, k1 = h ? kb : pk;
    const bool first = m0 >= m1;
    mx = first ? m0 : m1;
    return first ? k0 : k1;
}

// q . k in fp64 for this row: each lane sums its own dims (chunks 2 g + h,
// `chunk(g)` points at those 4 floats of the key), and the two halves are
// added (the same sum in both lanes).
// The query's fp64 copies are made afresh at every call (an empty volatile
// asm on each value keeps the compiler from hoisting 2 x 64 registers of
// them out of the key loop), and at most four chunks are read ahead, so the
// sum costs a few registers beside the kernels' live accumulators.
template <int NG, typename F>
__device__ __forceinline__ double exact_dot(const f32x4 (&qf)[NG], F chunk) {
    double acc = 0.0;
#pragma unroll
    for (int g0 = 0; g0 < NG; g0 += 4) {
        f32x4 kv[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) kv[g] = *reinterpret_cast<const f32x4 *>(chunk(g0 + g));
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                float qv = qf[g0 + g][s];
                asm volatile("" : "+v"(qv));
                acc = fma((double)qv, (double)kv[g][s], acc);
            }
    }
    return acc + __shfl_xor(acc, 32);
}

template <int DMAX, bool CAUSAL>
__device__ __forceinline__ void fa_tile_scores(const FaFused &p, const float *ks, const f32x4 (&qf)[DMAX / 8],
                                               int64_t k0, int64_t my_q, int lane, float (&sv)[16]) {
    constexpr int NG = DMAX / 8;
    constexpr int kStride = DMAX + 4;
    const int c = lane & 31, h = lane >> 5;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const f32x4 kf = *reinterpret_cast<const f32x4 *>(ks + c * kStride + 8 * g + 4 * h);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[s], qf[g][s], acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t key = k0 + attn::key_of(r, h);
        bool keep = key < p.sk;
        if (CAUSAL) keep = keep && key <= my_q;
        sv[r] = keep ? acc[r] * p.scale : -INFINITY;
    }
}

template <int DMAX, bool CAUSAL>
__global__ __launch_bounds__(kFaThreads, 2) void fa_fused_kernel(FaFused p) {
    using KvStage = attn::KvStage<DMAX, kFaThreads>;
    constexpr int NG = DMAX / 8, ND = DMAX / 32;
    constexpr int kStride = DMAX + 4;
    constexpr int kBKV = attn::kBKV;
    constexpr int kTile = kBKV * kStride;
    __shared__ __attribute__((aligned(16))) float lds[4 * kTile];  // K0 K1 V0 V1
    float *const lk = lds;
    float *const lv = lds + 2 * kTile;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, h = lane >> 5;
    const int64_t b = blockIdx.x;
    // Causal: heaviest query blocks first, and for a grid resident all at
    // once the light half in ascending order (as the SDPA kernel).
    int qb = (int)blockIdx.y;
    if (CAUSAL) {
        const int y = (int)blockIdx.y, half = (p.nqb + 1) / 2;
        qb = (p.fold && y >= half) ? y - half : p.nqb - 1 - y;
    }
    const int64_t q0 = (int64_t)qb * kFaBQ;
    const int64_t wq0 = q0 + wave * 32;
    const int64_t my_q = wq0 + c;
    const bool row_ok = my_q < p.sq;
    const float *Q = p.q + b * p.sq * p.d;
    const float *K = p.k + b * p.sk * p.d;
    const float *V = p.v + b * p.sk * p.d;
    double *mrow = p.mblk + (b * p.sq + (row_ok ? my_q : p.sq - 1)) * p.nbw;

    f32x4 qf[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int dim = 8 * g + 4 * h;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (row_ok && dim < p.d) v = *reinterpret_cast<const f32x4 *>(Q + my_q * p.d + dim);
        qf[g] = v;
    }

    const int64_t kv_end = CAUSAL ? min(p.sk, q0 + kFaBQ) : p.sk;
    const int64_t ntiles = (kv_end + kBKV - 1) / kBKV;

    // ---- pass 1: running max after every key block, and l ----
    KvStage gk, gv;
    gk.load(K, 0, p.sk, p.d, p.d, tid);
    gk.store(lk, tid);
    __syncthreads();
    double m = -INFINITY;  // exact running max
    float l = 0.f;
    for (int64_t t = 0; t < ntiles; ++t) {
        const int cur = t & 1;
        const bool more = t + 1 < ntiles;
        if (more) gk.load(K, (t + 1) * kBKV, p.sk, p.d, p.d, tid);
        const int64_t k0 = t * kBKV;
        if (!CAUSAL || k0 <= wq0 + 31) {
            float sv[16];
            const float *ks = lk + cur * kTile;
            fa_tile_scores<DMAX, CAUSAL>(p, ks, qf, k0, my_q, lane, sv);
            float mx;
            const int kw = tile_argmax(sv, h, mx);
            const double dot = exact_dot(qf, [&](int g) { return ks + kw * kStride + 8 * g + 4 * h; });
            const double m_new = mx != -INFINITY ? fmax(m, dot * (double)p.scale) : m;
            const bool dead = (m_new == -INFINITY);
            const float alpha = dead ? 1.f : __expf((float)(m - m_new));
            const float mn = (float)m_new;
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) ps += dead ? 0.f : __expf(sv[r] - mn);
            ps += __shfl_xor(ps, 32);
            l = l * alpha + ps;
            m = m_new;
        }
        // After a block's last tile m is that block's M_t.  Both halves of
        // the wave hold the same m and write it, so each lane later reads
        // back its own store.
        if ((k0 + kBKV) % p.bn == 0 || !more) {
            if (row_ok) mrow[k0 / p.bn] = m;
        }
        if (more) gk.store(lk + (cur ^ 1) * kTile, tid);
        __syncthreads();
    }

    // ---- pass 2: the weights from M, and O = W . V ----
    const int64_t jv = CAUSAL ? min(p.sk, my_q + 1) : p.sk;  // visible keys of this row
    const int64_t vb = (jv - 1) / p.bn;                         // last block with one
    const double m_v = m;
    const double m_v1 = vb >= 1 ? mrow[vb - 1] : 0.0;
    const double e_tail = vb >= 1 ? (double)min(p.bn, p.sk - vb * p.bn) * (m_v1 - m_v) : 0.0;
    f32x16 o[ND];
#pragma unroll
    for (int j = 0; j < ND; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.f;

    gk.load(K, 0, p.sk, p.d, p.d, tid);
    gv.load(V, 0, p.sk, p.d, p.d, tid);
    gk.store(lk, tid);
    gv.store(lv, tid);
    __syncthreads();
    for (int64_t t = 0; t < ntiles; ++t) {
        const int cur = t & 1;
        const bool more = t + 1 < ntiles;
        if (more) {
            gk.load(K, (t + 1) * kBKV, p.sk, p.d, p.d, tid);
            gv.load(V, (t + 1) * kBKV, p.sk, p.d, p.d, tid);
        }
        const int64_t k0 = t * kBKV;
        if (!CAUSAL || k0 <= wq0 + 31) {
            const int64_t blk = k0 / p.bn;
            const double mt64 = mrow[blk];
            const double mp64 = blk >= 1 ? mrow[blk - 1] : 0.0;
            float sv[16];
            fa_tile_scores<DMAX, CAUSAL>(p, lk + cur * kTile, qf, k0, my_q, lane, sv);
            const int64_t n = min(p.bn, p.sk - blk * p.bn);
            const float e = blk < vb ? (float)((double)p.bn * (mt64 - m_v1) + e_tail) : 0.f;
            const float delta = (float)(mp64 - mt64);
            const float mt = (float)mt64;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t idx = k0 + attn::key_of(r, h) - blk * p.bn;
                float w = 0.f;
                if (sv[r] != -INFINITY) {
                    if (blk == 0)
                        w = idx == n - 1 ? __expf((sv[r] - mt) + e) : 0.f;
                    else
                        w = __expf(((sv[r] - mt) + (float)(n - 1 - idx) * delta) + e);
                }
                sv[r] = w;
            }
            const float *vt = lv + cur * kTile;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float *vrow = vt + attn::key_of(r, h) * kStride + c;
#pragma unroll
                for (int j = 0; j < ND; ++j)
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * j], sv[r], o[j], 0, 0, 0);
            }
        }
        if (more) {
            gk.store(lk + (cur ^ 1) * kTile, tid);
            gv.store(lv + (cur ^ 1) * kTile, tid);
        }
        __syncthreads();
    }

    // O / l.  Lane (query c, half h), register r of block j holds head dim
    // 32 j + 8 (r / 4) + 4 h + r % 4.
    if (row_ok) {
        float *orow = p.out + (b * p.sq + my_q) * p.d;
#pragma unroll
        for (int j = 0; j < ND; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int dim = 32 * j + 8 * i + 4 * h;
                if (dim < p.d) {
                    f32x4 v = {o[j][4 * i] / l, o[j][4 * i + 1] / l, o[j][4 * i + 2] / l, o[j][4 * i + 3] / l};
                    *reinterpret_cast<f32x4 *>(orow + dim) = v;
                }
            }
    }
}

// ---- single-pass form (block_n = 32 or 64) ----------------------------------
//
// Block by block, the recurrence itself in closed form per block: with M_t
// the running max after block t and delta_t = M_{t-1} - M_t,
//   O <- O * exp(n_t delta_t) + sum_{j in t} exp((s_j - M_t) + (n_t - 1 - idx_j) delta_t) v_j
//   l <- l * exp(delta_t)     + sum_{j in t} exp(s_j - M_t)
// (block 0: only its last key enters O), and O / l at the end -- the same
// weights as the two-pass form, E_t now applied as the product of the later
// blocks' factors.  A 64-key block spans two 32-key tiles: the first tile's
// scores wait in registers until the second gives the block max.  K tiles
// are double-buffered and V tiles triple-buffered through LDS (tile u in V
// buffer u % 3), all requested straight into LDS one tile ahead; 80 KB per
// workgroup at d <= 128, two workgroups per CU.
template <int DMAX, bool CAUSAL>
__device__ __forceinline__ void fa_scores_lds(const FaFused &p, const float *ks, const f32x4 (&qf)[DMAX / 8],
                                              int64_t k0, int64_t my_q, int lane, float (&sv)[16]) {
    constexpr int NG = DMAX / 8;
    constexpr int kBKV = attn::kBKV;
    const int c = lane & 31, h = lane >> 5;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const f32x4 kf = attn::k_frag<DMAX>(ks, c, h, g);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[s], qf[g][s], acc, 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // MFMA
    }
    // keys k0 + i with i < lim are visible to this row
    int64_t lim64 = p.sk - k0;
    if (CAUSAL) lim64 = min(lim64, my_q - k0 + 1);
    const int lim = (int)max<int64_t>(0, min<int64_t>(lim64, kBKV));
#pragma unroll
    for (int r = 0; r < 16; ++r) sv[r] = attn::key_of(r, h) < lim ? acc[r] * p.scale : -INFINITY;
}

template <int DMAX, bool CAUSAL, int TPB>
__global__ __launch_bounds__(kFaThreads, 2) void fa_onepass_kernel(FaFused p) {
    static_assert(TPB == 1 || TPB == 2, "32- or 64-key blocks");
    constexpr int NG = DMAX / 8, ND = DMAX / 32;
    constexpr int kBKV = attn::kBKV;
    constexpr int kTile = kBKV * DMAX;
    constexpr int NVB = TPB + 1;  // V tile buffers
    using KL = attn::KvLds<DMAX, kFaThreads, false>;
    using VL = attn::KvLds<DMAX, kFaThreads, true>;
    __shared__ __attribute__((aligned(1024))) float lds[(2 + NVB) * kTile];
    float *const lk = lds;
    float *const lv = lds + 2 * kTile;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, h = lane >> 5;
    const int64_t b = blockIdx.x;
    int qb = (int)blockIdx.y;
    if (CAUSAL) {
        const int y = (int)blockIdx.y, half = (p.nqb + 1) / 2;
        qb = (p.fold && y >= half) ? y - half : p.nqb - 1 - y;
    }
    const int64_t q0 = (int64_t)qb * kFaBQ;
    const int64_t wq0 = q0 + wave * 32;
    const int64_t my_q = wq0 + c;
    const bool row_ok = my_q < p.sq;
    const float *Q = p.q + b * p.sq * p.d;
    const float *K = p.k + b * p.sk * p.d;
    const float *V = p.v + b * p.sk * p.d;

    f32x4 qf[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int dim = 8 * g + 4 * h;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (row_ok && dim < p.d) v = *reinterpret_cast<const f32x4 *>(Q + my_q * p.d + dim);
        qf[g] = v;
    }
    f32x16 o[ND];
#pragma unroll
    for (int j = 0; j < ND; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.f;
    double m = -INFINITY;  // exact running max
    float l = 0.f;
    float sa[16];  // scores of a two-tile block's first tile
#pragma unroll
    for (int r = 0; r < 16; ++r) sa[r] = -INFINITY;

    const int64_t kv_end = CAUSAL ? min(p.sk, q0 + kFaBQ) : p.sk;
    const int64_t ntiles = (kv_end + kBKV - 1) / kBKV;

    // Requests tile u (K and V) into its buffers.
    auto issue_k = [&](int64_t u) { KL::issue(K, u * kBKV, p.sk, p.d, p.d, lk + (u & 1) * kTile, wave, lane); };
    auto issue_v = [&](int64_t u) { VL::issue(V, u * kBKV, p.sk, p.d, p.d, lv + (u % NVB) * kTile, wave, lane); };
    auto issue = [&](int64_t u) {
        issue_k(u);
        issue_v(u);
    };
    // The exact score of key kw of K tile u for this row.
    auto exact_score = [&](int64_t u, int kw) {
        const float *ks = lk + (u & 1) * kTile;
        return exact_dot(qf, [&](int g) { return ks + (2 * g + h) * (4 * kBKV) + 4 * kw; }) * (double)p.scale;
    };
    // Scores of tile u into x; with EXACT also the exact value of this
    // row's largest one into ex (-inf without a visible key).
    auto scores = [&](int64_t u, float (&x)[16], double &ex, auto exact) {
        const int64_t k0 = u * kBKV;
        ex = -INFINITY;
        if (!CAUSAL || k0 <= wq0 + 31) {
            fa_scores_lds<DMAX, CAUSAL>(p, lk + (u & 1) * kTile, qf, k0, my_q, lane, x);
            if constexpr (decltype(exact)::value) {
                float mx;
                const int kw = tile_argmax(x, h, mx);
                const double e = exact_score(u, kw);
                if (mx != -INFINITY) ex = e;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) x[r] = -INFINITY;
        }
    };
    const std::true_type with_exact{};
    const std::false_type no_exact{};
    // Weights of tile u of block blk in place (scores in x); adds
    // exp(s - mt) of its visible keys to ps.
    auto weights = [&](float (&x)[16], int64_t u, int64_t blk, int64_t n, float mt, float delta, float &ps) {
        // key_of(r, h) = 4 h + kr, kr = 8 (r / 4) + r % 4; the key's
        // position in its block is base + 4 h + kr, so n - 1 - idx =
        // rest - kr with rest = n - 1 - base - 4 h (small integers, exact).
        const int base = (int)(u * kBKV - blk * p.bn);
        const int rest = (int)n - 1 - base - 4 * h;
        const float frest = (float)rest;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int kr = 8 * (r >> 2) + (r & 3);
            float w = 0.f;
            if (x[r] != -INFINITY) {
                const float e = __expf(x[r] - mt);
                ps += e;
                if (blk == 0)
                    w = rest == kr ? e : 0.f;
                else
                    w = __expf((x[r] - mt) + (frest - (float)kr) * delta);
            }
            x[r] = w;
        }
    };
    // O += W . V for tile u.  The scheduling groups keep the V reads a
    // step ahead of their MFMAs instead of hoisting all of them (which
    // would need 16 * ND registers at once).
    auto pv = [&](const float (&x)[16], int64_t u) {
        const float *vt = lv + (u % NVB) * kTile;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
#pragma unroll
            for (int j = 0; j < ND; ++j)
                o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(attn::v_elem<DMAX>(vt, attn::key_of(r, h), h, c, j), x[r],
                                                            o[j], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, ND / 2, 0);  // DS reads
            __builtin_amdgcn_sched_group_barrier(0x008, ND, 0);      // MFMA
        }
    };
    // Block blk from tiles u0 .. u0 + nt - 1 (nt = 1 or 2), their scores in
    // sa (first of two) and sv.
    // (bx: the block's exact max, -inf without a visible key)
    auto finish = [&](float (&sa_)[16], float (&sv_)[16], double bx, int64_t u0, int nt, int64_t blk) {
        const int64_t n = min(p.bn, p.sk - blk * p.bn);
        const double mt64 = fmax(m, bx);
        // Key 0 is visible to every row, so m is finite from block 1 on.
        const float delta = blk == 0 ? 0.f : (float)(m - mt64);
        const float mt = (float)mt64;
        float ps = 0.f;
        if (nt == 2) weights(sa_, u0, blk, n, mt, delta, ps);
        weights(sv_, u0 + nt - 1, blk, n, mt, delta, ps);
        ps += __shfl_xor(ps, 32);
        l = l * __expf(delta) + ps;
        m = mt64;
        const float corr = __expf((float)n * delta);
#pragma unroll
        for (int j = 0; j < ND; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][r] *= corr;
        if (nt == 2) pv(sa_, u0);
        pv(sv_, u0 + nt - 1);
    };
    // A wave whose last query precedes a tile's first key skips it.
    auto live = [&](int64_t u) { return !CAUSAL || u * kBKV <= wq0 + 31; };

    issue(0);
    attn::wait_vm0();
    __syncthreads();
    for (int64_t t = 0; t < ntiles; t += TPB) {
        const int64_t blk = t / TPB;
        float sv[16];
        if (TPB == 2 && t + 1 < ntiles) {
            // First tile of the block: scores wait in sa.  The block's
            // exact max is taken once, from its key with the largest fp32
            // score in either tile, so the first tile's K stays in its
            // buffer until every wave has that score: the next block's
            // first K tile (same buffer) is requested after a barrier.
            issue(t + 1);
            double unused;
            scores(t, sa, unused, no_exact);
            attn::wait_vm0();
            __syncthreads();
            if (t + 2 < ntiles) issue_v(t + 2);
            scores(t + 1, sv, unused, no_exact);
            float mxa, mxv;
            const int kwa = tile_argmax(sa, h, mxa);
            const int kwv = tile_argmax(sv, h, mxv);
            const bool first = mxa >= mxv;  // the same in both lanes of a row
            const double e = exact_score(first ? t : t + 1, first ? kwa : kwv);
            const double bx = (first ? mxa : mxv) != -INFINITY ? e : -INFINITY;
            __syncthreads();
            if (t + 2 < ntiles) issue_k(t + 2);
            if (live(t) || live(t + 1)) finish(sa, sv, bx, t, 2, blk);
        } else {
            if (t + 1 < ntiles) issue(t + 1);
            double bx;
            scores(t, sv, bx, with_exact);
            if (live(t)) finish(sa, sv, bx, t, 1, blk);
        }
        attn::wait_vm0();
        __syncthreads();
    }

    if (row_ok) {
        float *orow = p.out + (b * p.sq + my_q) * p.d;
#pragma unroll
        for (int j = 0; j < ND; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int dim = 32 * j + 8 * i + 4 * h;
                if (dim < p.d) {
                    f32x4 v = {o[j][4 * i] / l, o[j][4 * i + 1] / l, o[j][4 * i + 2] / l, o[j][4 * i + 3] / l};
                    *reinterpret_cast<f32x4 *>(orow + dim) = v;
                }
            }
    }
}

__global__ void fa_zero_kernel(float *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.f;
}

}  // namespace

int64_t flash_attention_max_blocks() { return 8192; }

// The fused form needs whole 32-key tiles per key block, head dims the
// 16-byte staging covers (d % 4 == 0, at most 128) and aligned operands.
bool flash_attention_fused_fits(const FlashAttnDesc &d) {
    return d.block_n % attn::kBKV == 0 && d.d > 0 && d.d <= 128 && d.d % 4 == 0 && aligned16(d.q) &&
           aligned16(d.k) && aligned16(d.v) && aligned16(d.out) && (d.sq + kFaBQ - 1) / kFaBQ <= 65535;
}

size_t flash_attention_workspace_bytes(const FlashAttnDesc &d) {
    if (d.sk > 0 && flash_attention_fused_fits(d))
        return sizeof(double) * (size_t)d.batch * (size_t)d.sq * (size_t)((d.sk + d.block_n - 1) / d.block_n);
    return sizeof(float) * (size_t)d.batch * (size_t)d.sq * (size_t)d.sk;
}

int launch_flash_attention_blockwise(const FlashAttnDesc &d, hipStream_t s) {
    if (d.batch == 0 || d.sq == 0 || d.d == 0) return GFH_SUCCESS;
    if (d.sk > 0 && flash_attention_fused_fits(d)) {
        FaFused p;
        p.q = d.q;
        p.k = d.k;
        p.v = d.v;
        p.out = d.out;
        p.mblk = reinterpret_cast<double *>(d.ws);
        p.sq = d.sq;
        p.sk = d.sk;
        p.d = d.d;
        p.bn = d.block_n;
        p.nbw = (d.sk + d.block_n - 1) / d.block_n;
        p.scale = d.scale;
        p.nqb = (int)((d.sq + kFaBQ - 1) / kFaBQ);
        p.fold = d.causal && d.batch * p.nqb <= 2 * (int64_t)device_cu_count();
        const dim3 grid((unsigned)d.batch, (unsigned)p.nqb), block(kFaThreads);
        if (d.block_n == 32 || d.block_n == 64) {
#define GFH_FA_ONEPASS(DM, TPB)                                                                  \
    do {                                                                                         \
        if (d.causal)                                                                            \
            hipLaunchKernelGGL((fa_onepass_kernel<DM, true, TPB>), grid, block, 0, s, p);        \
        else                                                                                     \
            hipLaunchKernelGGL((fa_onepass_kernel<DM, false, TPB>), grid, block, 0, s, p);       \
    } while (0)
            if (d.d <= 64) {
                if (d.block_n == 32)
                    GFH_FA_ONEPASS(64, 1);
                else
                    GFH_FA_ONEPASS(64, 2);
            } else {
                if (d.block_n == 32)
                    GFH_FA_ONEPASS(128, 1);
                else
                    GFH_FA_ONEPASS(128, 2);
            }
#undef GFH_FA_ONEPASS
            return check_launch("flash_attention (single pass)");
        }
        if (d.d <= 64) {
            if (d.causal)
                hipLaunchKernelGGL((fa_fused_kernel<64, true>), grid, block, 0, s, p);
            else
                hipLaunchKernelGGL((fa_fused_kernel<64, false>), grid, block, 0, s, p);
        } else {
            if (d.causal)
                hipLaunchKernelGGL((fa_fused_kernel<128, true>), grid, block, 0, s, p);
            else
                hipLaunchKernelGGL((fa_fused_kernel<128, false>), grid, block, 0, s, p);
        }
        return check_launch("flash_attention (fused)");
    }
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
        r.q = d.q;
        r.k = d.k;
        r.d = d.d;
        r.scale = d.scale;
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
