// kv_attention.hip -- attention of a few new queries over a key/value cache:
// the scaled_dot_product_attention step (ghostflow-nn/src/attention.rs:
// 11-49) of MultiHeadAttention::forward_with_cache (:100-144) at decode
// time, reading K/V where the cache keeps them.
//
// Layout: the reference's [B, S, E] projections with head h in columns
// h*D .. h*D+D-1 (reshape_for_attention, :146-150, is a view of exactly
// that): q (b, i, h, d) at q[b*q_bs + i*q_rs + h*D + d], and K/V (b, j, h, d)
// at k[b*kv_bs + j*kv_rs + h*D + d] -- for a cache of capacity C,
// kv_bs = C*E and kv_rs = E, so appending a step is writing rows in place
// instead of the reference's concat_tensors copy (:214-247).
//
// HBM-bound: every key and value row of a head (D floats) is read once per
// query block.  Work split (flash-decoding):
//  * workgroup = (b, h) x query block (up to QB = 4 queries) x key split;
//    256 threads = 8 half-waves of 32 lanes, lane l holding head dims
//    4l .. 4l+3, so one 16-byte load per lane reads a whole 512-byte row;
//  * half-wave w takes keys j0 + w, j0 + w + 8, ... of the split, kU of
//    them (K and V rows) in flight, and keeps the online-softmax state
//    (running max m, sum l, output accumulator) of each query; the dot
//    product is summed over the 32 lanes with xor shuffles, then scaled
//    (the scale multiplies the finished dot product, :24-25) and masked;
//  * the 8 half-wave states are merged through LDS; with several splits
//    each workgroup publishes (m, l, acc) with agent-scope stores and the
//    last of a (b, h, query block) to arrive (agent-scope counter) merges
//    the splits in split order -- deterministic, one launch -- and returns
//    the counter to 0.
// Masks as the reference: an explicit mask is cycled over the flattened
// [B, H, Sq, Skv] scores, m > 0.5 keeps (apply_attention_mask, :51-64);
// `causal` keeps key j for query i when j <= Skv - Sq + i (the query rows
// are the last Sq positions).  A query whose keys are all masked gets NaN,
// as the reference's softmax over all -inf does.  The weights output
// (nullable) receives softmax probabilities: raw scores are written as
// they are computed and normalized once the row's max and sum are known.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

namespace gfh {
namespace {

constexpr int kKvThreads = 256;
constexpr int kHalves = kKvThreads / 32;  // half-waves per workgroup
constexpr int kU = 4;                     // keys per half-wave in flight
constexpr int kPartStride = 132;          // floats per published query state: m, l, 2 pad, acc[128]

struct KvParams {
    const float *q, *k, *v;
    float *out, *weights;
    const float *mask;
    int64_t mask_numel;
    int64_t q_bs, q_rs, kv_bs, kv_rs, o_bs, o_rs;
    int64_t h, sq, kv_len, d;
    float scale;
    int causal;
    int nqb;
    int64_t nsplit, chunk;
    float *part;    // [bh][nqb][nsplit][QB][kPartStride]
    int *counters;  // [bh * nqb], zero at rest
};

template <int QB, bool WEIGHTS>
__global__ __launch_bounds__(kKvThreads, 2) void kv_attention_kernel(KvParams p) {
    __shared__ float red_m[kHalves][QB], red_l[kHalves][QB];
    __shared__ __attribute__((aligned(16))) float red_a[kHalves][QB][128];
    __shared__ float fin_m[QB], fin_l[QB];
    __shared__ int last_flag;

    const int tid = threadIdx.x, lane = tid & 31, half = tid >> 5;
    const int64_t split = blockIdx.x % p.nsplit;
    const int64_t rest = blockIdx.x / p.nsplit;
    const int qb = (int)(rest % p.nqb);
    const int64_t bh = rest / p.nqb;
    const int64_t b = bh / p.h, hh = bh % p.h;
    const int64_t i0 = (int64_t)qb * QB;
    const int nq = (int)min<int64_t>(QB, p.sq - i0);
    const int64_t j0 = split * p.chunk, j1 = min(j0 + p.chunk, p.kv_len);
    const int dim = 4 * lane;
    const bool dim_ok = dim < p.d;
    const int dimc = dim_ok ? dim : 0;  // lanes past D read dims 0..3 and are never stored

    const float *qbase = p.q + b * p.q_bs + hh * p.d + dimc;
    const float *kbase = p.k + b * p.kv_bs + hh * p.d + dimc;
    const float *vbase = p.v + b * p.kv_bs + hh * p.d + dimc;

    f32x4 qv[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(qbase + min<int64_t>(i0 + i, p.sq - 1) * p.q_rs);
        qv[i] = dim_ok ? v : f32x4{0.f, 0.f, 0.f, 0.f};  // zero dims past D add nothing to the dot product
    }
    float m[QB], l[QB];
    f32x4 acc[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.f;
        acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    for (int64_t jb = j0 + half; jb < j1; jb += kHalves * kU) {
        // Keys past the split re-read key jb (inside it) and are masked.
        f32x4 kr[kU], vr[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t j = jb + kHalves * u;
            const int64_t jc = j < j1 ? j : jb;
            kr[u] = *reinterpret_cast<const f32x4 *>(kbase + jc * p.kv_rs);
            vr[u] = *reinterpret_cast<const f32x4 *>(vbase + jc * p.kv_rs);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t j = jb + kHalves * u;
#pragma unroll
            for (int i = 0; i < QB; ++i) {
                float s = qv[i][0] * kr[u][0];
                s = fmaf(qv[i][1], kr[u][1], s);
                s = fmaf(qv[i][2], kr[u][2], s);
                s = fmaf(qv[i][3], kr[u][3], s);
#pragma unroll
                for (int off = 16; off > 0; off >>= 1) s += __shfl_xor(s, off);
                s = s * p.scale;
                const int64_t qi = i0 + i;
                bool keep = j < j1 && i < nq;
                if (p.causal) keep = keep && j <= p.kv_len - p.sq + qi;
                if (p.mask && keep) keep = p.mask[((bh * p.sq + qi) * p.kv_len + j) % p.mask_numel] > 0.5f;
                s = keep ? s : -INFINITY;
                if (WEIGHTS && lane == 0 && j < j1 && i < nq)
                    __hip_atomic_store(p.weights + (bh * p.sq + qi) * p.kv_len + j, s, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                const float m_new = fmaxf(m[i], s);
                if (m_new == -INFINITY) continue;  // every key so far masked (uniform over the half-wave)
                const float corr = __expf(m[i] - m_new);
                const float pj = __expf(s - m_new);
                l[i] = l[i] * corr + pj;
                acc[i] = acc[i] * corr + pj * vr[u];
                m[i] = m_new;
            }
        }
    }

    // Raw scores must be complete before any thread of the workgroup reads
    // them back for normalizing.
    if constexpr (WEIGHTS) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

    // Merge the half-waves.  Thread (i, lane) = (tid / 32, tid % 32) then
    // owns query i's dims 4 lane .. 4 lane + 3.
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        if (lane == 0) {
            red_m[half][i] = m[i];
            red_l[half][i] = l[i];
        }
        *reinterpret_cast<f32x4 *>(&red_a[half][i][dim]) = acc[i];
    }
    __syncthreads();
    const int qi_loc = tid >> 5;  // QB <= kHalves
    float M = -INFINITY, L = 0.f;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
    if (qi_loc < QB) {
#pragma unroll
        for (int w = 0; w < kHalves; ++w) M = fmaxf(M, red_m[w][qi_loc]);
#pragma unroll
        for (int w = 0; w < kHalves; ++w) {
            const float mw = red_m[w][qi_loc];
            const float f = mw == -INFINITY ? 0.f : __expf(mw - M);
            L = L + red_l[w][qi_loc] * f;
            A = A + *reinterpret_cast<const f32x4 *>(&red_a[w][qi_loc][dim]) * f;
        }
    }

    if (p.nsplit > 1) {
        // Publish this split's state, then count the arrival.
        if (qi_loc < QB) {
            float *dst = p.part + ((((bh * p.nqb + qb) * p.nsplit + split) * QB + qi_loc) * kPartStride);
            if (lane == 0) {
                __hip_atomic_store(dst, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(dst + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (dim_ok) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    __hip_atomic_store(dst + 4 + dim + e, A[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's stores are complete
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(p.counters + bh * p.nqb + qb, 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            last_flag = (old == (int)p.nsplit - 1);
        }
        __syncthreads();
        if (!last_flag) return;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // Merge the splits in split order.
        M = -INFINITY;
        L = 0.f;
        A = f32x4{0.f, 0.f, 0.f, 0.f};
        if (qi_loc < QB) {
            const float *src = p.part + (((bh * p.nqb + qb) * p.nsplit) * QB + qi_loc) * kPartStride;
            for (int64_t s = 0; s < p.nsplit; ++s)
                M = fmaxf(M, __hip_atomic_load(src + s * QB * kPartStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            for (int64_t s = 0; s < p.nsplit; ++s) {
                const float *ps = src + s * QB * kPartStride;
                const float ms = __hip_atomic_load(ps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float f = ms == -INFINITY ? 0.f : __expf(ms - M);
                L = L + __hip_atomic_load(ps + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * f;
                if (dim_ok) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        A[e] = A[e] +
                               __hip_atomic_load(ps + 4 + dim + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * f;
                }
            }
        }
        if (tid == 0)
            __hip_atomic_store(p.counters + bh * p.nqb + qb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // out = acc / l.  A row with every key masked has M = -inf, L = 0 and
    // A = 0: 0 / 0 gives the reference's NaN.
    if (qi_loc < nq && dim_ok) {
        const float inv = 1.0f / L;
        float *orow = p.out + b * p.o_bs + (i0 + qi_loc) * p.o_rs + hh * p.d + dim;
        *reinterpret_cast<f32x4 *>(orow) = A * inv;
    }
    if constexpr (WEIGHTS) {
        // Normalize the whole row [0, kv_len) of each query of the block
        // (written by every split; visible at agent scope).
        if (qi_loc < QB && lane == 0) {
            fin_m[qi_loc] = M;
            fin_l[qi_loc] = L;
        }
        __syncthreads();
        for (int64_t t = tid; t < (int64_t)nq * p.kv_len; t += kKvThreads) {
            const int i = (int)(t / p.kv_len);
            const int64_t j = t % p.kv_len;
            float *w = p.weights + (bh * p.sq + i0 + i) * p.kv_len + j;
            const float s = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *w = __expf(s - fin_m[i]) / fin_l[i];
        }
    }
}

template <int QB>
int launch_qb(const KvParams &p, int64_t blocks, bool weights, hipStream_t s) {
    const dim3 grid((unsigned)blocks), block(kKvThreads);
    if (weights)
        hipLaunchKernelGGL((kv_attention_kernel<QB, true>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((kv_attention_kernel<QB, false>), grid, block, 0, s, p);
    return check_launch("kv_attention");
}

}  // namespace

int launch_kv_attention(const KvAttnDesc &d, hipStream_t s) {
    KvParams p{};
    p.q = d.q;
    p.k = d.k;
    p.v = d.v;
    p.out = d.out;
    p.weights = d.weights;
    p.mask = d.mask;
    p.mask_numel = d.mask_numel;
    p.q_bs = d.q_bs;
    p.q_rs = d.q_rs;
    p.kv_bs = d.kv_bs;
    p.kv_rs = d.kv_rs;
    p.o_bs = d.o_bs;
    p.o_rs = d.o_rs;
    p.h = d.h;
    p.sq = d.sq;
    p.kv_len = d.kv_len;
    p.d = d.d;
    p.scale = d.scale;
    p.causal = d.causal ? 1 : 0;
    // Queries per block: up to 4 (8 would need twice the registers and
    // halve the occupancy); longer query runs take several blocks, each
    // reading the keys again (mostly from L2).
    const int qb = d.sq == 1 ? 1 : d.sq == 2 ? 2 : 4;
    p.nqb = (int)((d.sq + qb - 1) / qb);
    // Split the keys so that there are about 512 workgroups (two per CU),
    // each taking at least 64 keys.
    const int64_t bhq = d.b * d.h * p.nqb;
    const int64_t want = std::max<int64_t>(1, (512 + bhq - 1) / bhq);
    int64_t chunk = (d.kv_len + want - 1) / want;
    chunk = std::max<int64_t>(64, (chunk + 31) & ~(int64_t)31);
    p.chunk = chunk;
    p.nsplit = (d.kv_len + chunk - 1) / chunk;
    if (p.nsplit > 1) {
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(float) * (size_t)(bhq * p.nsplit * qb * kPartStride), &ws));
        p.part = static_cast<float *>(ws);
        GFH_TRY(stream_counters(s, (size_t)bhq, &p.counters));
    }
    const int64_t blocks = bhq * p.nsplit;
    if (blocks > 0x7fffffff) return set_error(GFH_INVALID_SHAPE, "kv_attention: grid too large");
    const bool w = d.weights != nullptr;
    if (qb == 1) return launch_qb<1>(p, blocks, w, s);
    if (qb == 2) return launch_qb<2>(p, blocks, w, s);
    return launch_qb<4>(p, blocks, w, s);
}

}  // namespace gfh
