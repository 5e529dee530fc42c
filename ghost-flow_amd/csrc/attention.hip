// attention.hip -- fused scaled-dot-product attention and row softmax on
// CDNA4 f32 MFMA.
//
// Computes, per (batch, head) slice, softmax(mask(Q K^T * scale)) V -- the
// work of scaled_dot_product_attention (ghostflow-nn/src/attention.rs:11-49)
// and ops::attention::flash_attention (ghostflow-cuda/src/ops.rs:166-224) --
// without materializing the score matrix, using the online-softmax
// recurrence (running max m, running sum l, rescale by exp(m_old - m_new)),
// the blockwise form of ghostflow-nn/src/flash_attention.rs:178-250.
//
// Semantics kept from the reference:
//   * the scale multiplies the finished dot product (mul_scalar after the
//     matmul, attention.rs:24-25);
//   * causal masking is j > i -> -inf (ops.rs:205-224); an explicit mask is
//     cycled over the flattened scores, m > 0.5 keeps (attention.rs:51-64);
//   * a row whose scores are all -inf yields NaN, as softmax over all -inf
//     does in the reference (max = -inf, exp(NaN)).
//
// Two kernels: sdpa_set_kernel (below) for every call without a weights
// output -- 16-query sets on 16x16x4 MFMAs, light and heavy causal query
// groups paired per SIMD, four waves per SIMD -- and sdpa_fwd_kernel, which
// also writes the [sq, skv] weights.  sdpa_fwd_kernel's layout (one
// 256-thread workgroup = 4 wave64s per 128 queries of one (b, h); K/V
// streamed in 32-key tiles through double-buffered LDS):
//   * S^T = K . Q^T on v_mfma_f32_32x32x2_f32: keys are the MFMA rows and
//     queries the columns, so lane l owns query l%32 and holds 16 of the 32
//     keys of a tile (the other 16 sit in lane l^32).  Row max / row sum are
//     in-register folds plus one cross-half shuffle.
//   * Q for the wave's 32 queries stays in registers for the whole key loop
//     (one 16-byte fragment per 8 head dims).
//   * O^T = V^T . P^T on the same MFMA: the B operand of step r is exactly
//     accumulator register r of S^T (same key, same query), so P never moves;
//     the A operand is one conflict-free ds_read_b32 of V per step.
//   * O accumulators (head_dim/32 blocks of 16 registers) are per-lane per
//     query, so the online-softmax rescale is a per-lane multiply.
//   * Causal: key tiles above the diagonal are skipped (per workgroup and per
//     wave), and workgroups are issued heaviest query block first.  The
//     (b,h) index is the fastest grid dimension, so all query blocks of one
//     (b,h) land on the same XCD and share its K/V in that L2.
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

constexpr int kThreads = 256;
constexpr int kBQ = 128;  // queries per workgroup (32 per wave)
constexpr int kBKV = attn::kBKV;  // keys per LDS tile

// Element (b, h, i, d) of q is at q[b*q_bs + h*q_hs + i*q_rs + d] (K, V with
// the kv_* strides, the output with o_*): [B, H, S, D] contiguous, or the
// [B, S, E] projections with heads as column blocks (h stride D, row stride
// E) that MultiHeadAttention attends over without a transpose.  weights is
// always [B*H, sq, skv].
struct SdpaParams {
    const float *q, *k, *v;
    float *out;
    float *weights;
    const float *mask;
    int64_t mask_numel;
    int64_t q_bs, q_hs, q_rs, kv_bs, kv_hs, kv_rs, o_bs, o_hs, o_rs;
    int64_t h;
    int64_t sq, skv, d;
    int64_t bh;
    int64_t causal_off;  // causal keeps key j for query i when j <= i + causal_off
    float scale;
    int nqb;
    int fold;  // causal issue order for a grid that is resident all at once (below)
};

using attn::key_of;
template <int DMAX>
using KvStage = attn::KvStage<DMAX, kThreads>;

// Scaled, masked scores of one 32-key tile for this lane's query.
template <int DMAX, bool CAUSAL, bool MASK>
__device__ __forceinline__ void tile_scores(const SdpaParams &p, const float *ks, const f32x4 (&qf)[DMAX / 8],
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
        const int64_t key = k0 + key_of(r, h);
        float v = acc[r] * p.scale;
        bool keep = key < p.skv;
        if (CAUSAL) keep = keep && key <= my_q + p.causal_off;
        if (MASK && keep) {
            const int64_t f = ((int64_t)blockIdx.x * p.sq + my_q) * p.skv + key;
            keep = p.mask[f % p.mask_numel] > 0.5f;
        }
        sv[r] = keep ? v : -INFINITY;
    }
}

// Two workgroups per CU (at most 256 registers per lane): with one, every
// softmax, LDS and barrier stall of a wave left its SIMD's MFMA idle --
// B=4, H=32, D=128 causal at S=2048: 1487 us with 243 VGPRs + 64 AGPRs, one
// wave per SIMD; 1287 us with 249 VGPRs, two.
template <int DMAX, bool CAUSAL, bool MASK, bool WEIGHTS>
__global__ __launch_bounds__(kThreads, 2) void sdpa_fwd_kernel(SdpaParams p) {
    constexpr int NG = DMAX / 8, ND = DMAX / 32;
    constexpr int kStride = DMAX + 4;
    constexpr int kTile = kBKV * kStride;
    __shared__ __attribute__((aligned(16))) float lds[4 * kTile];  // K0 K1 V0 V1
    float *const lk = lds;
    float *const lv = lds + 2 * kTile;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, h = lane >> 5;
    const int64_t bh = blockIdx.x;
    // Causal issue order.  Query block qb walks qb + 1 key blocks, so the
    // heaviest go first; when the whole grid is resident at once (two
    // workgroups per CU), workgroups j and j + #CUs share a CU, and the
    // second half of the y range then runs the light blocks in ascending
    // order, pairing the heaviest with the lightest (B=4, H=32, S=512: CU
    // loads 16 + 4 and 12 + 8 key blocks instead of 16 + 8 and 12 + 4).
    int qb = (int)blockIdx.y;
    if (CAUSAL) {
        const int y = (int)blockIdx.y, half = (p.nqb + 1) / 2;
        qb = (p.fold && y >= half) ? y - half : p.nqb - 1 - y;
    }
    const int64_t q0 = (int64_t)qb * kBQ;
    const int64_t wq0 = q0 + wave * 32;
    const int64_t my_q = wq0 + c;
    const int64_t bb = bh / p.h, hh = bh % p.h;
    const float *Q = p.q + bb * p.q_bs + hh * p.q_hs;
    const float *K = p.k + bb * p.kv_bs + hh * p.kv_hs;
    const float *V = p.v + bb * p.kv_bs + hh * p.kv_hs;

    f32x4 qf[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int dim = 8 * g + 4 * h;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (my_q < p.sq && dim < p.d) v = *reinterpret_cast<const f32x4 *>(Q + my_q * p.q_rs + dim);
        qf[g] = v;
    }

    f32x16 o[ND];
#pragma unroll
    for (int j = 0; j < ND; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.f;
    float m = -INFINITY, l = 0.f;

    const int64_t kv_end = CAUSAL ? min(p.skv, q0 + kBQ + p.causal_off) : p.skv;
    const int64_t ntiles = (kv_end + kBKV - 1) / kBKV;

    KvStage<DMAX> gk, gv;
    if (ntiles > 0) {
        gk.load(K, 0, p.skv, p.d, p.kv_rs, tid);
        gv.load(V, 0, p.skv, p.d, p.kv_rs, tid);
        gk.store(lk, tid);
        gv.store(lv, tid);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int64_t t = 0; t < ntiles; ++t) {
        const int cur = t & 1;
        const bool more = t + 1 < ntiles;
        if (more) {
            gk.load(K, (t + 1) * kBKV, p.skv, p.d, p.kv_rs, tid);
            gv.load(V, (t + 1) * kBKV, p.skv, p.d, p.kv_rs, tid);
        }
        const int64_t k0 = t * kBKV;
        // A wave whose last query precedes the tile's first key has nothing to do.
        const bool active = !CAUSAL || k0 <= wq0 + 31 + p.causal_off;
        if (active) {
            float sv[16];
            tile_scores<DMAX, CAUSAL, MASK>(p, lk + cur * kTile, qf, k0, my_q, lane, sv);
            float mb = sv[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mb = fmaxf(mb, sv[r]);
            mb = fmaxf(mb, __shfl_xor(mb, 32));
            const float m_new = fmaxf(m, mb);
            const bool dead = (m_new == -INFINITY);  // every score so far masked
            const float alpha = dead ? 1.f : __expf(m - m_new);
            float psum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                sv[r] = dead ? 0.f : __expf(sv[r] - m_new);
                psum += sv[r];
            }
            psum += __shfl_xor(psum, 32);
            l = l * alpha + psum;
            m = m_new;
#pragma unroll
            for (int j = 0; j < ND; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
            const float *vt = lv + cur * kTile;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float *vrow = vt + key_of(r, h) * kStride + c;
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

    // O = O / l.  Lane (query c, half h), register r of block j holds head
    // dim 32j + 8(r/4) + 4h + r%4: four consecutive dims per 16-byte store.
    if (my_q < p.sq) {
        const float inv_l = 1.0f / l;
        float *orow = p.out + bb * p.o_bs + hh * p.o_hs + my_q * p.o_rs;
#pragma unroll
        for (int j = 0; j < ND; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int dim = 32 * j + 8 * i + 4 * h;
                if (dim < p.d) {
                    f32x4 v = {o[j][4 * i] * inv_l, o[j][4 * i + 1] * inv_l, o[j][4 * i + 2] * inv_l,
                               o[j][4 * i + 3] * inv_l};
                    *reinterpret_cast<f32x4 *>(orow + dim) = v;
                }
            }
    }

    if constexpr (WEIGHTS) {
        // Second pass: the normalized probabilities exp(s - m) / l for every
        // key (masked ones come out as 0), written as the [sq, skv] weights.
        const int64_t wtiles = (p.skv + kBKV - 1) / kBKV;
        const float inv_l = 1.0f / l;
        float *wrow = p.weights + (bh * p.sq + (my_q < p.sq ? my_q : 0)) * p.skv;
        __syncthreads();
        for (int64_t t = 0; t < wtiles; ++t) {
            gk.load(K, t * kBKV, p.skv, p.d, p.kv_rs, tid);
            gk.store(lk, tid);
            __syncthreads();
            float sv[16];
            tile_scores<DMAX, CAUSAL, MASK>(p, lk, qf, t * kBKV, my_q, lane, sv);
            if (my_q < p.sq) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t key = t * kBKV + 8 * i + 4 * h;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (key + e < p.skv) wrow[key + e] = __expf(sv[4 * i + e] - m) * inv_l;
                }
            }
            __syncthreads();
        }
    }
}

// ---- balanced 16-query sets (no weights output) ------------------------------
//
// The same recurrence over 16-query sets on v_mfma_f32_16x16x4_f32 (same
// rate per SIMD as the 32x32x2 form), one set per wave, eight waves per
// workgroup.  The query groups of a (b, h) slice (G = ceil(sq / 16)) are
// paired as (G - 1 - p, p): waves 0-3 take the light groups p = 4 blockIdx.y
// + w, waves 4-7 the heavy groups G - 1 - p.  Under causal masking a pair
// covers about (sq + 32) / 32 (16-query x 32-key) tile units whatever p is,
// so every workgroup, and every SIMD (waves w and w + 4 share one), carries
// the same load; with 32-query waves over 128-query blocks the heaviest
// blocks set the critical path.  One set needs at most 128 registers, so two
// 64 KB workgroups per CU put four waves on each SIMD, which hides the
// softmax, LDS and barrier stalls that two waves per SIMD left exposed
// (B=4, H=32, D=128 causal: S=512 88 us, S=2048 1.14 ms; with two sets per
// wave and two waves per SIMD, 91 us and 1.17 ms).
//
// Fragment layouts (lane l, c = l % 16, quarter h = l / 16):
//  * S^T = K . Q^T: A = K (row = key, k = dim), B = Q^T.  The four dims a
//    lane supplies over steps e = 0..3 of dim group u are 16u + 4h + e, so a
//    lane's K and Q operands for a group are one 16-byte read each.  The
//    accumulator of key block kb (keys 16kb .. 16kb + 15) holds, in register
//    r, key 16kb + 4h + r for query c.
//  * O^T = V^T . P^T: step r of key block kb takes key 16kb + 4h + r in
//    quarter h, so its B operand is register r of that block's scores and P
//    never moves; the A operand is V[key][16b + c], one ds_read_b32.
//  * O block b (dims 16b .. 16b + 15): lane holds dims 16b + 4h + r of query c.
//  * K and V tiles are requested straight into LDS (global_load_lds, no
//    staging registers).  K is chunk-major (16-byte chunk q of key r at slot
//    32q + r: a fragment read is 256 contiguous bytes per quarter); V is
//    key-major with chunk q of key r at q ^ (4 * bits 2-3 of r), so the four
//    quarters of a V read (keys 4 apart, 16 dims each) fall on disjoint
//    16-bank groups: quarter h finds dims 16b .. 16b + 15 at 16 (b ^ h).
constexpr int kSetQ = 16;  // queries per set
constexpr int kSetThreads = 512;

template <int DMAX>
struct QuerySet {
    static constexpr int NU = DMAX / 16;  // 16-dim groups
    f32x4 qf[NU];
    f32x4 o[NU];
    float m, l;
    int q;       // this lane's query
    int kv_end;  // keys this set reads (causal: up to its last query)
    bool valid;
};

// One 32-key tile for a set.  kq = this lane's K fragment base; vb[j] = its
// V base for the dim blocks b with b % 4 == j (the quarter swizzle above).
template <int DMAX, bool CAUSAL, bool MASK>
__device__ __forceinline__ void set_tile(const SdpaParams &p, QuerySet<DMAX> &st, const float *kq,
                                         const float *(&vb)[4], int k0, int h) {
    constexpr int NU = DMAX / 16;
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    // The MFMA phases run at raised wave priority, so that another wave of
    // the SIMD in its softmax does not delay their issue.
    __builtin_amdgcn_s_setprio(1);
    // K fragments one dim group ahead of the MFMAs that use them: chunk
    // 4u + h of key 16kb + c (kq already holds h and c).
    auto kfrag = [&](int u, int kb) { return *reinterpret_cast<const f32x4 *>(kq + 4 * (128 * u + 16 * kb)); };
    f32x4 kf[2][2];
    kf[0][0] = kfrag(0, 0);
    kf[0][1] = kfrag(0, 1);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        if (u + 1 < NU) {
            kf[(u + 1) & 1][0] = kfrag(u + 1, 0);
            kf[(u + 1) & 1][1] = kfrag(u + 1, 1);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of these MFMAs
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[u & 1][kb][e], st.qf[u][e], acc[kb], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);

    // Scale, mask, online softmax.  lim = the last key of the tile the query
    // keeps, relative to k0 (clamped to the tile: 32-bit comparisons).
    int last = (int)p.skv - 1;
    if (CAUSAL) last = min(last, st.q + (int)p.causal_off);
    const int lim = max(-1, min(kBKV, last - k0));
    float pv[8];
    float mb = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int j = 16 * (i >> 2) + 4 * h + (i & 3);
        const float v = acc[i >> 2][i & 3] * p.scale;
        bool keep = j <= lim;
        if (MASK && keep) {
            const int64_t f = ((int64_t)blockIdx.x * p.sq + st.q) * p.skv + (k0 + j);
            keep = p.mask[f % p.mask_numel] > 0.5f;
        }
        pv[i] = keep ? v : -INFINITY;
        mb = fmaxf(mb, pv[i]);
    }
    const float m_new = fmaxf(st.m, quarter_max(mb));
    const bool dead = (m_new == -INFINITY);  // every score so far masked
    const float alpha = dead ? 1.f : __expf(st.m - m_new);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        pv[i] = dead ? 0.f : __expf(pv[i] - m_new);
        psum += pv[i];
    }
    st.l = st.l * alpha + quarter_sum(psum);
    st.m = m_new;
#pragma unroll
    for (int b = 0; b < NU; ++b) st.o[b] *= alpha;

    // P.V step i = 4 kb + r: key 16kb + 4h + r (4h is in vb), dim 16b + c;
    // the V elements of step i + 1 are read while step i's MFMAs run.
    auto vload = [&](int i, float (&va)[NU]) {
#pragma unroll
        for (int b = 0; b < NU; ++b) va[b] = vb[b & 3][(16 * (i >> 2) + (i & 3)) * DMAX + 64 * (b >> 2)];
    };
    __builtin_amdgcn_s_setprio(1);
    float va[2][NU];
    vload(0, va[0]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (i + 1 < 8) vload(i + 1, va[(i + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < NU; ++b)
            st.o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[i & 1][b], pv[i], st.o[b], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
}

// At most 128 registers per lane (the second bound is waves per SIMD):
// two workgroups per CU, four waves per SIMD.
template <int DMAX, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(kSetThreads, 4) void sdpa_set_kernel(SdpaParams p) {
    static_assert(DMAX == 64 || DMAX == 128, "direct-to-LDS tiles cover 64 or 128 dims");
    constexpr int NU = DMAX / 16;
    constexpr int kTile = kBKV * DMAX;
    using KLoad = attn::KvLds<DMAX, kSetThreads, false>;
    using VLoad = attn::KvLds<DMAX, kSetThreads, true>;
    __shared__ __attribute__((aligned(16))) float lds[4 * kTile];  // K0 K1 V0 V1
    float *const lk = lds;
    float *const lv = lds + 2 * kTile;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: set bounds and LDS targets in SGPRs
    const int c = lane & 15, h = lane >> 4;
    const int64_t bh = blockIdx.x;
    const int64_t bb = bh / p.h, hh = bh % p.h;
    const float *Q = p.q + bb * p.q_bs + hh * p.q_hs;
    const float *K = p.k + bb * p.kv_bs + hh * p.kv_hs;
    const float *V = p.v + bb * p.kv_bs + hh * p.kv_hs;

    // Indices are 32-bit (the launcher requires sq, skv < 2^31).  The heavy
    // wave holds group G - 1 - pair (the middle group of an odd G included),
    // the light wave group pair when it is smaller; neither exists for pairs
    // past the last.
    const int sq = (int)p.sq, skv = (int)p.skv;
    const int ngroups = (sq + kSetQ - 1) / kSetQ;
    const int pair = (int)blockIdx.y * 4 + (wave & 3);
    const bool heavy = wave >= 4;
    auto kv_end_of = [&](int g) -> int {
        return CAUSAL ? min(skv, min((g + 1) * kSetQ, sq) + (int)p.causal_off) : skv;
    };
    QuerySet<DMAX> st;
    const int g = heavy ? ngroups - 1 - pair : pair;
    st.valid = heavy ? ngroups - 1 - pair >= pair : ngroups - 1 - pair > pair;
    st.q = g * kSetQ + c;
    st.kv_end = kv_end_of(g);
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int dim = 16 * u + 4 * h;
        // Branch-free: a clamped address, zero where there is no query or dim.
        const bool in = st.valid && st.q < sq && dim < p.d;
        const int64_t row = st.valid ? min(st.q, sq - 1) : 0;
        const f32x4 v = *reinterpret_cast<const f32x4 *>(Q + row * p.q_rs + (dim < p.d ? dim : 0));
        st.qf[u] = in ? v : f32x4{0.f, 0.f, 0.f, 0.f};
        st.o[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // The workgroup streams the keys of its heaviest set: wave 4's.
    const int kv_end = kv_end_of(ngroups - 1 - (int)blockIdx.y * 4);
    const int ntiles = (kv_end + kBKV - 1) / kBKV;

    if (ntiles > 0) {
        KLoad::issue(K, 0, skv, p.d, p.kv_rs, lk, wave, lane);
        VLoad::issue(V, 0, skv, p.d, p.kv_rs, lv, wave, lane);
    }
    attn::wait_vm0();
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int cur = t & 1;
        // The other buffers were last read before the previous barrier.
        if (t + 1 < ntiles) {
            KLoad::issue(K, (t + 1) * kBKV, skv, p.d, p.kv_rs, lk + (cur ^ 1) * kTile, wave, lane);
            VLoad::issue(V, (t + 1) * kBKV, skv, p.d, p.kv_rs, lv + (cur ^ 1) * kTile, wave, lane);
        }
        const int k0 = t * kBKV;
        const float *kq = lk + cur * kTile + 4 * (32 * h + c);
        const float *vt = lv + cur * kTile + 4 * h * DMAX + c;
        const float *vb[4] = {vt + 16 * (0 ^ h), vt + 16 * (1 ^ h), vt + 16 * (2 ^ h), vt + 16 * (3 ^ h)};
        if (st.valid && k0 < st.kv_end) set_tile<DMAX, CAUSAL, MASK>(p, st, kq, vb, k0, h);
        attn::wait_vm0();
        __syncthreads();
    }

    // O = O / l; lane (query c, quarter h) holds dims 16b + 4h .. + 3.
    if (st.valid && st.q < sq) {
        const float inv_l = 1.0f / st.l;
        float *orow = p.out + bb * p.o_bs + hh * p.o_hs + (int64_t)st.q * p.o_rs;
#pragma unroll
        for (int b = 0; b < NU; ++b) {
            const int dim = 16 * b + 4 * h;
            if (dim < p.d) *reinterpret_cast<f32x4 *>(orow + dim) = st.o[b] * inv_l;
        }
    }
}

// ---- row softmax (Tensor::softmax(-1)) ---------------------------------------
// Per row, as activation.rs:188-212: a max fold from -inf (NaN-ignoring, like
// f32::max), the sum of exp(x - max), then exp(x - max) / sum with a true
// division.  expf is ROCm's full-precision device expf.  The sum is taken in
// a different order than the reference's ascending one (within its rounding
// bound); the max is exact in any order.
//
// Rows of up to 4096 columns (cols % 4 == 0, 16-byte aligned): one wave per
// row, the row held in registers between the passes, so x is read once and y
// written once (8 bytes per element); 16-byte loads, NV per lane.
// Longer rows: one workgroup per row, x read twice.
// Both walk the rows with a grid stride, so any row count fits one launch.
constexpr int kSoftmaxGrid = 8 * 1024;  // workgroups: 32 per CU

// NT: nontemporal loads and stores, for inputs that do not stay in the
// 256 MB MALL anyway (chosen by the launcher).
template <int NV, bool NT>
__global__ __launch_bounds__(kThreads) void softmax_rows_wave_kernel(const float *__restrict__ x,
                                                                     float *__restrict__ y, int64_t rows,
                                                                     int64_t cols) {
    const int lane = threadIdx.x & 63;
    const int64_t nwaves = (int64_t)gridDim.x * (kThreads / 64);
    for (int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); row < rows; row += nwaves) {
        const float *xr = x + row * cols;
        float *yr = y + row * cols;
        f32x4 v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int64_t c = 4 * (lane + 64 * i);
            const f32x4 *src = reinterpret_cast<const f32x4 *>(xr + c);
            v[i] = c < cols ? (NT ? __builtin_nontemporal_load(src) : *src)
                            : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        }
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) mx = fmaxf(mx, v[i][e]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        // exp, then a pairwise sum inside the lane (log2(4 NV) levels) and
        // across the wave: the rounding error grows with the tree depth,
        // not with the row length.
        float part[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = expf(v[i][e] - mx);
            part[i] = 4 * (lane + 64 * i) < cols ? (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]) : 0.f;
        }
#pragma unroll
        for (int w = 1; w < NV; w *= 2)
#pragma unroll
            for (int i = 0; i + w < NV; i += 2 * w) part[i] += part[i + w];
        const float sum = wave_sum(part[0]);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int64_t c = 4 * (lane + 64 * i);
            if (c < cols) {
                f32x4 *dst = reinterpret_cast<f32x4 *>(yr + c);
                if (NT)
                    __builtin_nontemporal_store(v[i] / sum, dst);
                else
                    *dst = v[i] / sum;
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void softmax_rows_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                               int64_t rows, int64_t cols) {
    __shared__ float red[kThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const float *xr = x + row * cols;
        float *yr = y + row * cols;

        float mx = -INFINITY;
        for (int64_t i = threadIdx.x; i < cols; i += kThreads) mx = fmaxf(mx, xr[i]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        if (lane == 0) red[wave] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();

        float sum = 0.f;
        for (int64_t i = threadIdx.x; i < cols; i += kThreads) sum += expf(xr[i] - mx);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        if (lane == 0) red[wave] = sum;
        __syncthreads();
        sum = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();  // red is rewritten by the next row

        for (int64_t i = threadIdx.x; i < cols; i += kThreads) yr[i] = expf(xr[i] - mx) / sum;
    }
}

template <int DMAX, bool CAUSAL, bool MASK>
void launch_sdpa_variant(const SdpaParams &p, dim3 grid, bool weights, hipStream_t s) {
    if (weights)
        hipLaunchKernelGGL((sdpa_fwd_kernel<DMAX, CAUSAL, MASK, true>), grid, dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL((sdpa_fwd_kernel<DMAX, CAUSAL, MASK, false>), grid, dim3(kThreads), 0, s, p);
}

// Head dims up to 32 run the 64-dim tiles (the direct-to-LDS loader's
// smallest row).
template <int DMAX, bool CAUSAL>
void launch_sdpa_sets(const SdpaParams &p, bool mask, hipStream_t s) {
    constexpr int DP = DMAX < 64 ? 64 : DMAX;
    const int64_t groups = (p.sq + kSetQ - 1) / kSetQ;
    const int64_t pairs = (groups + 1) / 2;
    const dim3 grid((unsigned)p.bh, (unsigned)((pairs + 3) / 4));
    if (mask)
        hipLaunchKernelGGL((sdpa_set_kernel<DP, CAUSAL, true>), grid, dim3(kSetThreads), 0, s, p);
    else
        hipLaunchKernelGGL((sdpa_set_kernel<DP, CAUSAL, false>), grid, dim3(kSetThreads), 0, s, p);
}

template <int DMAX>
void launch_sdpa_d(const SdpaParams &p, dim3 grid, bool causal, bool mask, bool weights, hipStream_t s) {
    // The balanced kernel serves every call without a weights output whose
    // indices fit 32 bits; the 32-query kernel writes the weights.
    constexpr int64_t kMax32 = (int64_t)1 << 31;
    if (!weights && p.sq + p.causal_off < kMax32 && p.skv < kMax32 - kBKV) {
        if (causal)
            launch_sdpa_sets<DMAX, true>(p, mask, s);
        else
            launch_sdpa_sets<DMAX, false>(p, mask, s);
        return;
    }
    if (causal) {
        if (mask)
            launch_sdpa_variant<DMAX, true, true>(p, grid, weights, s);
        else
            launch_sdpa_variant<DMAX, true, false>(p, grid, weights, s);
    } else {
        if (mask)
            launch_sdpa_variant<DMAX, false, true>(p, grid, weights, s);
        else
            launch_sdpa_variant<DMAX, false, false>(p, grid, weights, s);
    }
}

}  // namespace

int launch_softmax_lastdim(const float *x, float *y, int64_t rows, int64_t cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return GFH_SUCCESS;
    if (cols % 4 == 0 && cols <= 4096 && aligned16(x) && aligned16(y)) {
        const int64_t wgs = std::min<int64_t>((rows + kThreads / 64 - 1) / (kThreads / 64), kSoftmaxGrid);
        const dim3 grid((unsigned)wgs), block(kThreads);
        const int nv = (int)((cols / 4 + 63) / 64);  // f32x4 per lane
        // Nontemporal access when x and y together exceed the MALL: at
        // [262144, 2048] (4.3 GB) 777 against 809 us per call (a plain device
        // copy of the same bytes takes 870-950 us), while at [65536, 512]
        // (268 MB, which stays in the MALL between calls) it took 42.2
        // against 39.5 us.
        const bool nt = (double)rows * (double)cols * 8.0 > 256.0 * 1024 * 1024;
        auto go = [&](auto ntc) {
            constexpr bool NT = decltype(ntc)::value;
            if (nv <= 1)
                hipLaunchKernelGGL((softmax_rows_wave_kernel<1, NT>), grid, block, 0, s, x, y, rows, cols);
            else if (nv <= 2)
                hipLaunchKernelGGL((softmax_rows_wave_kernel<2, NT>), grid, block, 0, s, x, y, rows, cols);
            else if (nv <= 4)
                hipLaunchKernelGGL((softmax_rows_wave_kernel<4, NT>), grid, block, 0, s, x, y, rows, cols);
            else if (nv <= 8)
                hipLaunchKernelGGL((softmax_rows_wave_kernel<8, NT>), grid, block, 0, s, x, y, rows, cols);
            else
                hipLaunchKernelGGL((softmax_rows_wave_kernel<16, NT>), grid, block, 0, s, x, y, rows, cols);
        };
        if (nt)
            go(std::true_type{});
        else
            go(std::false_type{});
    } else {
        const dim3 grid((unsigned)std::min<int64_t>(rows, kSoftmaxGrid));
        hipLaunchKernelGGL(softmax_rows_kernel, grid, dim3(kThreads), 0, s, x, y, rows, cols);
    }
    return check_launch("softmax_lastdim");
}

int launch_sdpa(const SdpaDesc &d, hipStream_t s) {
    if (!aligned16(d.q) || !aligned16(d.k) || !aligned16(d.v) || !aligned16(d.out))
        return set_error(GFH_INVALID_DATA, "sdpa: q, k, v and out must be 16-byte aligned");
    SdpaParams p{};
    p.q = d.q;
    p.k = d.k;
    p.v = d.v;
    p.out = d.out;
    p.weights = d.weights;
    p.mask = d.mask;
    p.mask_numel = d.mask_numel;
    p.sq = d.sq;
    p.skv = d.skv;
    p.d = d.d;
    p.h = d.h;
    p.bh = d.b * d.h;
    if (d.strided) {
        p.q_bs = d.q_bs, p.q_hs = d.q_hs, p.q_rs = d.q_rs;
        p.kv_bs = d.kv_bs, p.kv_hs = d.kv_hs, p.kv_rs = d.kv_rs;
        p.o_bs = d.o_bs, p.o_hs = d.o_hs, p.o_rs = d.o_rs;
    } else {
        p.q_hs = d.sq * d.d, p.q_bs = d.h * p.q_hs, p.q_rs = d.d;
        p.kv_hs = d.skv * d.d, p.kv_bs = d.h * p.kv_hs, p.kv_rs = d.d;
        p.o_hs = p.q_hs, p.o_bs = p.q_bs, p.o_rs = d.d;
    }
    p.causal_off = d.causal ? d.skv - d.sq : 0;
    p.scale = d.scale;
    p.nqb = (int)((d.sq + kBQ - 1) / kBQ);
    p.fold = d.causal && p.bh * p.nqb <= 2 * (int64_t)device_cu_count();
    dim3 grid((unsigned)p.bh, (unsigned)p.nqb);
    const bool mask = d.mask != nullptr, weights = d.weights != nullptr;
    if (d.d <= 32)
        launch_sdpa_d<32>(p, grid, d.causal, mask, weights, s);
    else if (d.d <= 64)
        launch_sdpa_d<64>(p, grid, d.causal, mask, weights, s);
    else
        launch_sdpa_d<128>(p, grid, d.causal, mask, weights, s);
    return check_launch("sdpa");
}

}  // namespace gfh
