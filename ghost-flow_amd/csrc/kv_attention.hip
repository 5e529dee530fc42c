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
// HBM-bound: every key and value row is read once per query block.  Work
// split (flash-decoding):
//  * workgroup = (b, group of 8 heads) x query block (up to QB = 4
//    queries) x key split; 256 threads = 8 half-waves of 32 lanes, half-wave
//    w owning head 8g + w and lane l its dims 4l .. 4l+3.  For each key the
//    workgroup reads 8 adjacent 512-byte head slices of the cache row, 4 KB
//    contiguous (a read-only probe of this pattern streamed the 268 MB cache
//    of B=4, H=32, S=2048 in 45 us against 47-51 us for one head per
//    workgroup);
//  * each half-wave walks all keys of the split, kU of them (K and V rows)
//    in flight, keeping its head's online-softmax state (running max m,
//    sum l, output accumulator) per query; the dot product is summed over
//    the 32 lanes (DPP and readlane, no LDS), then scaled (the scale
//    multiplies the finished dot product, :24-25) and masked;
//  * with several splits each workgroup publishes its heads' (m, l, acc)
//    with agent-scope stores, and the last of a (b, head group, query
//    block) to arrive (agent-scope counter) merges the splits in split
//    order -- deterministic, one launch -- and returns the counter to 0.
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

// Every f32 product and sum is its own rounding, as in the reference CPU
// path (no FMA contraction).
#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kKvThreads = 256;
constexpr int kHalves = kKvThreads / 32;  // half-waves (heads) per workgroup
constexpr int kU = 8;                     // keys per half-wave in flight
constexpr int kPartStride = 132;          // floats per published query state: m, l, 2 pad, acc[128]

struct KvParams {
    const float *q, *k, *v;
    float *out, *weights;
    const float *mask;
    int64_t mask_numel;
    int64_t q_bs, q_rs, kv_bs, kv_rs, o_bs, o_rs;
    int64_t h, sq, kv_len, d;
    int64_t ngroups;  // head groups of kHalves
    float scale;
    int causal;
    int nqb;
    int64_t nsplit, chunk;
    float *part;    // [b*h][nqb][nsplit][QB][kPartStride]
    int *counters;  // [b * ngroups * nqb], zero at rest
};

template <int QB, bool WEIGHTS>
__global__ __launch_bounds__(kKvThreads, 2) void kv_attention_kernel(KvParams p) {
    __shared__ int last_flag;
    const int tid = threadIdx.x, lane = tid & 31, half = tid >> 5;
    const int64_t split = blockIdx.x % p.nsplit;
    const int64_t rest = blockIdx.x / p.nsplit;
    const int qb = (int)(rest % p.nqb);
    const int64_t bg = rest / p.nqb;
    const int64_t b = bg / p.ngroups;
    const int64_t hh = (bg % p.ngroups) * kHalves + half;
    const bool head_ok = hh < p.h;                 // uniform per half-wave
    const int64_t bh = b * p.h + (head_ok ? hh : p.h - 1);
    const int64_t hc = bh - b * p.h;               // this half-wave's head (clamped; never stored if past H)
    const int64_t i0 = (int64_t)qb * QB;
    const int nq = (int)min<int64_t>(QB, p.sq - i0);
    const int64_t j0 = split * p.chunk, j1 = min(j0 + p.chunk, p.kv_len);
    const int dim = 4 * lane;
    const bool dim_ok = dim < p.d;
    const int dimc = dim_ok ? dim : 0;  // lanes past D read dims 0..3 and are never stored

    const float *qbase = p.q + b * p.q_bs + hc * p.d + dimc;
    const float *kbase = p.k + b * p.kv_bs + hc * p.d + dimc;
    const float *vbase = p.v + b * p.kv_bs + hc * p.d + dimc;

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

    for (int64_t jb = j0; jb < j1; jb += kU) {
        // Keys past the split re-read its last key and are masked.
        f32x4 kr[kU], vr[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t jc = min(jb + u, j1 - 1);
            kr[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(kbase + jc * p.kv_rs));
            vr[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(vbase + jc * p.kv_rs));
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t j = jb + u;
#pragma unroll
            for (int i = 0; i < QB; ++i) {
                float s = qv[i][0] * kr[u][0];
                s = fmaf(qv[i][1], kr[u][1], s);
                s = fmaf(qv[i][2], kr[u][2], s);
                s = fmaf(qv[i][3], kr[u][3], s);
                s = half_wave_sum(s) * p.scale;
                const int64_t qi = i0 + i;
                bool keep = j < j1 && i < nq;
                if (p.causal) keep = keep && j <= p.kv_len - p.sq + qi;
                if (p.mask && keep) keep = p.mask[((bh * p.sq + qi) * p.kv_len + j) % p.mask_numel] > 0.5f;
                s = keep ? s : -INFINITY;
                if (WEIGHTS && head_ok && lane == 0 && j < j1 && i < nq)
                    __hip_atomic_store(p.weights + (bh * p.sq + qi) * p.kv_len + j, s, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                const float m_new = fmaxf(m[i], s);
                if (m_new == -INFINITY) continue;  // every key so far masked (uniform over the half-wave)
                const float corr = __expf(m[i] - m_new);
                const float pj = __expf(s - m_new);
                // explicit FMAs: this file does not contract a * b + c
                l[i] = fmaf(l[i], corr, pj);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][e] = fmaf(acc[i][e], corr, pj * vr[u][e]);
                m[i] = m_new;
            }
        }
    }

    if (p.nsplit > 1) {
        // Publish this split's state of each (head, query), then count the
        // workgroup's arrival.
        if (head_ok) {
#pragma unroll
            for (int i = 0; i < QB; ++i) {
                float *dst = p.part + (((bh * p.nqb + qb) * p.nsplit + split) * QB + i) * kPartStride;
                if (lane == 0) {
                    __hip_atomic_store(dst, m[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(dst + 1, l[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (dim_ok) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        __hip_atomic_store(dst + 4 + dim + e, acc[i][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        // split-K arrival protocol (common.hpp): steps 2-4
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's stores (and raw scores) are complete
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(p.counters + bg * p.nqb + qb, 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            last_flag = (old == (int)p.nsplit - 1);
        }
        __syncthreads();
        if (!last_flag) return;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // Merge the splits of each (head, query) in split order, online
        // (running max, rescaled sum and accumulator).  The states are
        // requested kG splits at a time before any is used, so the merge
        // costs a memory latency per kG splits, not per split.
        constexpr int kG = 8;
        if (head_ok) {
#pragma unroll
            for (int i = 0; i < QB; ++i) {
                const float *src = p.part + ((bh * p.nqb + qb) * p.nsplit * QB + i) * kPartStride;
                float M = -INFINITY, L = 0.f;
                f32x4 A = {0.f, 0.f, 0.f, 0.f};
                for (int64_t sp0 = 0; sp0 < p.nsplit; sp0 += kG) {
                    float ms[kG], ls[kG];
                    f32x4 as[kG];
#pragma unroll
                    for (int g = 0; g < kG; ++g) {
                        // past the last split: re-read it, then ignore it
                        const float *ps = src + min<int64_t>(sp0 + g, p.nsplit - 1) * QB * kPartStride;
                        ms[g] = __hip_atomic_load(ps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        ls[g] = __hip_atomic_load(ps + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            as[g][e] = __hip_atomic_load(ps + 4 + dimc + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
#pragma unroll
                    for (int g = 0; g < kG; ++g) {
                        if (sp0 + g >= p.nsplit || ms[g] == -INFINITY) continue;  // nothing kept in that split
                        const float M_new = fmaxf(M, ms[g]);
                        const float fo = __expf(M - M_new), fn = __expf(ms[g] - M_new);  // exp(-inf) = 0
                        L = L * fo + ls[g] * fn;
                        A = A * fo + as[g] * fn;
                        M = M_new;
                    }
                }
                m[i] = M;
                l[i] = L;
                acc[i] = A;
            }
        }
        if (tid == 0) __hip_atomic_store(p.counters + bg * p.nqb + qb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (WEIGHTS) {
        // The raw scores this workgroup wrote are read back below.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    if (!head_ok) return;

    // out = acc / l.  A row with every key masked has m = -inf, l = 0 and
    // acc = 0: 0 / 0 gives the reference's NaN.
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        if (i < nq && dim_ok) {
            float *orow = p.out + b * p.o_bs + (i0 + i) * p.o_rs + hc * p.d + dim;
            *reinterpret_cast<f32x4 *>(orow) = acc[i] * (1.0f / l[i]);
        }
    }
    if constexpr (WEIGHTS) {
        // Normalize this head's rows [0, kv_len) (written by every split,
        // visible at agent scope).
#pragma unroll
        for (int i = 0; i < QB; ++i) {
            if (i >= nq) continue;
            float *wrow = p.weights + (bh * p.sq + i0 + i) * p.kv_len;
            for (int64_t j = lane; j < p.kv_len; j += 32) {
                const float sc = __hip_atomic_load(wrow + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wrow[j] = __expf(sc - m[i]) / l[i];
            }
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
    p.ngroups = (d.h + kHalves - 1) / kHalves;
    // Split the keys so that there are about 256 workgroups (one per CU),
    // each taking at least 32 keys.  Measured at B=4, H=32, 2048 keys (16
    // head groups): 54.2 us with 16 splits and 8 keys in flight per
    // half-wave, against 56.1 us with 4 keys, 64.6-67.7 us with 32 splits
    // (the merge of the last arriver grows with the splits) and 71.8-89.7 us
    // with 8 (too few workgroups to stream).
    const int64_t gq = d.b * p.ngroups * p.nqb;
    const int64_t want = std::max<int64_t>(1, (256 + gq - 1) / gq);
    int64_t chunk = (d.kv_len + want - 1) / want;
    chunk = std::max<int64_t>(32, (chunk + kU - 1) / kU * kU);
    p.chunk = chunk;
    p.nsplit = (d.kv_len + chunk - 1) / chunk;
    if (p.nsplit > 1) {
        void *ws = nullptr;
        const size_t states = (size_t)(d.b * d.h) * (size_t)p.nqb * (size_t)p.nsplit * (size_t)qb;
        GFH_TRY(stream_workspace(s, sizeof(float) * states * kPartStride, &ws));
        p.part = static_cast<float *>(ws);
        GFH_TRY(stream_counters(s, (size_t)gq, &p.counters));
    }
    const int64_t blocks = gq * p.nsplit;
    if (blocks > 0x7fffffff) return set_error(GFH_INVALID_SHAPE, "kv_attention: grid too large");
    const bool w = d.weights != nullptr;
    if (qb == 1) return launch_qb<1>(p, blocks, w, s);
    if (qb == 2) return launch_qb<2>(p, blocks, w, s);
    return launch_qb<4>(p, blocks, w, s);
}

}  // namespace gfh
