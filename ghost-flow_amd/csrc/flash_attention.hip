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
//   * fa_set_kernel (block_n = 32 or 64): the recurrence per key block in
//     closed form, one pass, on 16-query sets (below);
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
// workgroup at d <= 128.
//
// Laid out as the balanced SDPA kernel:
// 16-query sets on v_mfma_f32_16x16x4_f32, one set per wave, eight waves per
// workgroup.  The query groups of a batch element (G = ceil(sq / 16)) are
// paired as (G - 1 - p, p): waves 0-3 take the light groups p = 4 blockIdx.y
// + w, waves 4-7 the heavy groups G - 1 - p, so under causal masking every
// workgroup and every SIMD (waves w and w + 4 share one) carries the same
// load.  A set walks the key blocks up to the one holding its last visible
// key (blocks past it are fully masked for every row of the set and change
// neither M nor O).  At most 128 registers per lane: two 80 KB workgroups
// per CU, four waves per SIMD.
//
// Per lane (c = l % 16, quarter h = l / 16): dims 16u + 4h .. + 3 of query c
// for the scores (S^T = K . Q^T), keys 16kb + 4h + r of a tile in score
// register 4kb + r, dims 16b + 4h + r of the output.  The block's exact max
// is the fp64 q . k of the query's largest fp32 score (its four lanes agree
// on the key: quarter_argmax), each lane summing its own 8 x 4 dims and the
// four partial sums added in a fixed order.  K tiles are chunk-major, V
// tiles key-major with the 4-way swizzle of the quarter reads.
constexpr int kFaSetThreads = 512;

template <int DMAX, bool CAUSAL, int TPB>
__global__ __launch_bounds__(kFaSetThreads, 4) void fa_set_kernel(FaFused p) {
    static_assert(TPB == 1 || TPB == 2, "32- or 64-key blocks");
    constexpr int NU = DMAX / 16;
    constexpr int kBKV = attn::kBKV;
    constexpr int kTile = kBKV * DMAX;
    constexpr int NVB = TPB + 1;  // V tile buffers
    using KL = attn::KvLds<DMAX, kFaSetThreads, false>;
    using VL = attn::KvLds<DMAX, kFaSetThreads, true>;
    __shared__ __attribute__((aligned(1024))) float lds[(2 + NVB) * kTile];
    float *const lk = lds;
    float *const lv = lds + 2 * kTile;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, h = lane >> 4;
    const int64_t b = blockIdx.x;
    // 32-bit indices: the entry point bounds sq below 2^31 and sk to 8192
    // key blocks (at most 2^19 keys with block_n <= 64)
    const int sq = (int)p.sq, sk = (int)p.sk, bn = (int)p.bn;
    const int ngroups = (sq + 15) / 16;
    const int pair = (int)blockIdx.y * 4 + (wave & 3);
    const bool heavy = wave >= 4;
    const int g = heavy ? ngroups - 1 - pair : pair;
    const bool valid = heavy ? ngroups - 1 - pair >= pair : ngroups - 1 - pair > pair;
    const int my_q = 16 * g + c;
    const int last_q = min(16 * g + 15, sq - 1);  // the set's last query
    auto blocks_of = [&](int gg) {
        const int end = CAUSAL ? min(sk, min(16 * gg + 16, sq)) : sk;
        return (end + bn - 1) / bn;
    };
    const int my_blocks = valid ? blocks_of(g) : 0;
    const int ntiles = min((sk + kBKV - 1) / kBKV, blocks_of(ngroups - 1 - (int)blockIdx.y * 4) * TPB);
    const float *Q = p.q + b * p.sq * p.d;
    const float *K = p.k + b * p.sk * p.d;
    const float *V = p.v + b * p.sk * p.d;

    f32x4 qf[NU], o[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int dim = 16 * u + 4 * h;
        // Branch-free: a clamped address, zero where there is no query or dim.
        const bool in = valid && my_q < sq && dim < p.d;
        const int64_t row = valid ? min(my_q, sq - 1) : 0;
        const f32x4 v = *reinterpret_cast<const f32x4 *>(Q + row * p.d + (dim < p.d ? dim : 0));
        qf[u] = in ? v : f32x4{0.f, 0.f, 0.f, 0.f};
        o[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    double m = -INFINITY;  // exact running max
    float l = 0.f;

    // The requests' per-lane addresses are recomputed at every call (a few
    // VALU ops per tile): hoisted out of the key loop they would hold two
    // registers per request for the whole loop, which this kernel's 128
    // cannot spare.
    auto fresh_lane = [&]() {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        return ln;
    };
    auto issue_k = [&](int u) {
        KL::issue(K, u * kBKV, p.sk, p.d, p.d, lk + (u & 1) * kTile, wave, fresh_lane());
    };
    auto issue_v = [&](int u) {
        VL::issue(V, u * kBKV, p.sk, p.d, p.d, lv + (u % NVB) * kTile, wave, fresh_lane());
    };
    auto issue = [&](int u) {
        issue_k(u);
        issue_v(u);
    };
    // Scores of tile u (scaled; -inf where the key is not visible).
    auto scores = [&](int u, float (&x)[8]) {
        const int k0 = u * kBKV;
        if (CAUSAL && k0 > last_q) {  // past every query of the set
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = -INFINITY;
            return;
        }
        // lane-derived values recomputed here (a reload from scratch in the
        // loop would also wait for the tiles in flight)
        int ln = (int)__lane_id();
        asm volatile("" : "+v"(ln));
        const int h = ln >> 4, c = ln & 15;
        const float *kq = lk + (u & 1) * kTile + 4 * (32 * h + c);
        auto kfrag = [&](int uu, int kb) { return *reinterpret_cast<const f32x4 *>(kq + 4 * (128 * uu + 16 * kb)); };
        f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        __builtin_amdgcn_s_setprio(1);
        f32x4 kf[2][2];
        kf[0][0] = kfrag(0, 0);
        kf[0][1] = kfrag(0, 1);
#pragma unroll
        for (int uu = 0; uu < NU; ++uu) {
            if (uu + 1 < NU) {
                kf[(uu + 1) & 1][0] = kfrag(uu + 1, 0);
                kf[(uu + 1) & 1][1] = kfrag(uu + 1, 1);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of these MFMAs
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[uu & 1][kb][e], qf[uu][e], acc[kb], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        // keys k0 + j with j < lim are visible to this row
        int lim = sk - k0;
        if (CAUSAL) lim = min(lim, 16 * g + c - k0 + 1);  // this row's query + 1 - k0
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int j = 16 * (i >> 2) + 4 * h + (i & 3);
            x[i] = j < lim ? acc[i >> 2][i & 3] * p.scale : -INFINITY;
        }
    };
    // This row's largest fp32 score over the block's NT tiles and its key
    // in the block (the same in the query's four lanes); the exact score of
    // that key (tile t0 + key / 32), or -inf without a visible key.
    auto block_max = [&](const float (&xa)[8], const float (&xb)[8], auto ntc, int t0) -> double {
        constexpr int NT = decltype(ntc)::value;
        // lane, quarter and column recomputed here (cheaper than holding
        // them through the loop, where a reload from scratch would also wait
        // for the tiles in flight)
        int ln = (int)__lane_id();
        asm volatile("" : "+v"(ln));
        const int h = ln >> 4;
        float mv = -INFINITY;
        int mk = 0;
#pragma unroll
        for (int ti = 0; ti < NT; ++ti)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = ti == 0 && NT == 2 ? xa[i] : xb[i];
                if (x > mv) {  // keys rise with (ti, i): ties keep the smaller
                    mv = x;
                    mk = 32 * ti + 16 * (i >> 2) + 4 * h + (i & 3);
                }
            }
        quarter_argmax(mv, mk, ln);
        const float *ks = lk + ((t0 + (mk >> 5)) & 1) * kTile;
        const int kw = mk & 31;
        // this lane's dims: chunk 4u + h of key kw at slot (4u + h) * 32 + kw
        double acc = 0.0;
#pragma unroll
        for (int u0 = 0; u0 < NU; u0 += 2) {
            f32x4 kv[2];
#pragma unroll
            for (int uu = 0; uu < 2; ++uu)
                kv[uu] = *reinterpret_cast<const f32x4 *>(ks + 4 * ((4 * (u0 + uu) + h) * 32 + kw));
#pragma unroll
            for (int uu = 0; uu < 2; ++uu)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float qv = qf[u0 + uu][e];
                    asm volatile("" : "+v"(qv));  // fp64 copies made here, not hoisted out of the key loop
                    acc = fma((double)qv, (double)kv[uu][e], acc);
                }
        }
        const double ex = quarter_sum_f64(acc, ln) * (double)p.scale;
        return mv == -INFINITY ? -INFINITY : ex;
    };
    // Weights of tile u of block blk in place (scores in x); adds exp(s - mt)
    // of its visible keys to ps.  The key's position in its block is
    // base + 16kb + 4h + r, so n - 1 - idx = rest - (16kb + r) with
    // rest = n - 1 - base - 4h (small integers, exact in fp32).
    auto weights = [&](float (&x)[8], int u, int blk, int n, float mt, float delta, float &ps) {
        const int rest = n - 1 - (u * kBKV - blk * bn) - 4 * h;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int kr = 16 * (i >> 2) + (i & 3);
            float w = 0.f;
            if (x[i] != -INFINITY) {
                const float e = __expf(x[i] - mt);
                ps += e;
                if (blk == 0)
                    w = rest == kr ? e : 0.f;
                else
                    w = __expf((x[i] - mt) + (float)(rest - kr) * delta);
            }
            x[i] = w;
        }
    };
    // O += W . V for tile u: step i = 4kb + r takes key 16kb + 4h + r and
    // dim 16b + c (quarter h finds dim block b at 16 (b ^ h) of the
    // swizzled row); the V elements of step i + 1 are read during step i.
    auto pv = [&](const float (&x)[8], int u) {
        const float *vt = lv + (u % NVB) * kTile + 4 * h * DMAX + c;
        const float *vb[4] = {vt + 16 * (0 ^ h), vt + 16 * (1 ^ h), vt + 16 * (2 ^ h), vt + 16 * (3 ^ h)};
        auto vload = [&](int i, float (&va)[NU]) {
#pragma unroll
            for (int bb = 0; bb < NU; ++bb) va[bb] = vb[bb & 3][(16 * (i >> 2) + (i & 3)) * DMAX + 64 * (bb >> 2)];
        };
        __builtin_amdgcn_s_setprio(1);
        float va[2][NU];
        vload(0, va[0]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i + 1 < 8) vload(i + 1, va[(i + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int bb = 0; bb < NU; ++bb)
                o[bb] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[i & 1][bb], x[i], o[bb], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    };
    // Block blk from tiles u0 .. u0 + NT - 1, scores in xa (first of two)
    // and xb, exact block max bx.
    auto finish = [&](float (&xa)[8], float (&xb)[8], double bx, int u0, auto ntc, int blk) {
        constexpr int NT = decltype(ntc)::value;
        const int n = min(bn, sk - blk * bn);
        const double mt64 = fmax(m, bx);
        // Key 0 is visible to every row, so m is finite from block 1 on.
        const float delta = blk == 0 ? 0.f : (float)(m - mt64);
        const float mt = (float)mt64;
        float ps = 0.f;
        if (NT == 2) weights(xa, u0, blk, n, mt, delta, ps);
        weights(xb, u0 + NT - 1, blk, n, mt, delta, ps);
        l = l * __expf(delta) + quarter_sum(ps);
        m = mt64;
        const float corr = __expf((float)n * delta);
#pragma unroll
        for (int bb = 0; bb < NU; ++bb) o[bb] *= corr;
        if (NT == 2) pv(xa, u0);
        pv(xb, u0 + NT - 1);
    };
    const std::integral_constant<int, 1> one{};
    const std::integral_constant<int, 2> two{};

    if (ntiles > 0) issue(0);
    attn::wait_vm0();
    __syncthreads();
    // Whole blocks of TPB tiles, then (TPB = 2) a last block of one tile.
    // Every wave passes the same barriers; a wave whose set ends earlier
    // only requests its share of the tiles.
    int t = 0;
    for (; t + TPB <= ntiles; t += TPB) {
        const int blk = t / TPB;
        const bool mine = blk < my_blocks;
        float xa[8], xb[8];
        if constexpr (TPB == 2) {
            // The block's exact max needs both tiles' scores, and its K
            // tiles stay in their buffers until every wave has it: the next
            // block's first K tile (same buffer as this block's first) is
            // requested after a barrier.
            issue(t + 1);
            if (mine) scores(t, xa);
            attn::wait_vm0();
            __syncthreads();
            if (t + 2 < ntiles) issue_v(t + 2);
            double bx = -INFINITY;
            if (mine) {
                scores(t + 1, xb);
                bx = block_max(xa, xb, two, t);
            }
            __syncthreads();
            if (t + 2 < ntiles) issue_k(t + 2);
            if (mine) finish(xa, xb, bx, t, two, blk);
        } else {
            if (t + 1 < ntiles) issue(t + 1);
            if (mine) {
                scores(t, xb);
                const double bx = block_max(xb, xb, one, t);
                finish(xb, xb, bx, t, one, blk);
            }
        }
        attn::wait_vm0();
        __syncthreads();
    }
    if (TPB == 2 && t < ntiles) {  // the last block holds one tile (its keys end the sequence)
        float xb[8];
        if (t / TPB < my_blocks) {
            scores(t, xb);
            const double bx = block_max(xb, xb, one, t);
            finish(xb, xb, bx, t, one, t / TPB);
        }
    }

    if (valid && my_q < sq) {
        float *orow = p.out + (b * p.sq + my_q) * p.d;
#pragma unroll
        for (int bb = 0; bb < NU; ++bb) {
            const int dim = 16 * bb + 4 * h;
            if (dim < p.d) *reinterpret_cast<f32x4 *>(orow + dim) = o[bb] / l;
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
            const int64_t groups = (d.sq + 15) / 16;
            const dim3 sgrid((unsigned)d.batch, (unsigned)(((groups + 1) / 2 + 3) / 4)), sblock(kFaSetThreads);
#define GFH_FA_ONEPASS(DM, TPB)                                                                  \
    do {                                                                                         \
        if (d.causal)                                                                            \
            hipLaunchKernelGGL((fa_set_kernel<DM, true, TPB>), sgrid, sblock, 0, s, p);          \
        else                                                                                     \
            hipLaunchKernelGGL((fa_set_kernel<DM, false, TPB>), sgrid, sblock, 0, s, p);         \
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
