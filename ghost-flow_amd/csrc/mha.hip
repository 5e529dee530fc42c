// mha.hip -- MultiHeadAttention::forward_with_cache
// (ghostflow-nn/src/attention.rs:100-144) on the device, host-side
// orchestration of the kernels of this library on one stream:
//
//   q = query . Wq^T + bq                      -> workspace [b*sq, e]
//   k_cache[:, past:past+sk] = key . Wk^T + bk   (the reference's concat of
//   v_cache[:, past:past+sk] = value . Wv^T + bv  past and new keys, :116-119,
//                                                  done by writing in place)
//   attn = softmax(mask(q . K^T * scale)) . V  over cache rows [0, past+sk)
//                                              -> workspace [b*sq, e]
//   out = attn . Wo^T + bo
//
// The projections are launch_sgemm NT calls (the row-dot GEMV up to 4 rows,
// the skinny MFMA GEMM up to 64, the MFMA tile GEMM beyond), with q, k and v
// in one grouped launch up to 64 rows when their shapes agree.  Attention reads q, K and V in the
// [B, S, E] layout where head h is a block of columns -- the storage of the
// reference's reshape_for_attention view (:146-150) -- with the decode
// kernel (kv_attention.hip) for up to 16 queries and the tiled SDPA kernel
// (attention.hip, strided) beyond; its output lands directly in the merged
// [B, S, E] order that reshape_from_attention (:152-157) produces.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace gfh {

size_t mha_workspace_bytes(int64_t b, int64_t sq, int64_t e) {
    const size_t one = ((size_t)b * (size_t)sq * (size_t)e * 4 + 255) & ~(size_t)255;
    return 2 * one;
}

int launch_mha_forward(const MhaDesc &d, void *workspace, hipStream_t s) {
    const int64_t e = d.e, hd = d.e / d.h;
    const size_t one = mha_workspace_bytes(d.b, d.sq, e) / 2;
    float *qbuf = static_cast<float *>(workspace);
    float *abuf = reinterpret_cast<float *>(static_cast<char *>(workspace) + one);

    auto linear_desc = [&](const float *x, int64_t m, const float *w, const float *bias, float *y, int64_t ldc) {
        SgemmDesc g;
        g.trans_b = true;
        g.m = m;
        g.n = e;
        g.k = e;
        g.a = x;
        g.lda = e;
        g.b = w;
        g.ldb = e;
        g.c = y;
        g.ldc = ldc;
        g.bias = bias;
        return g;
    };
    // New keys / values into cache rows [past, past + sk) of every batch.
    auto cache_desc = [&](const float *x, const float *w, const float *bias, float *cache) {
        float *dst = cache + d.past_len * e;
        if (d.sk == 1)  // one row per batch: rows e apart in x, capacity*e apart in the cache
            return linear_desc(x, d.b, w, bias, dst, d.capacity * e);
        if (d.b == 1 || d.capacity == d.sk)  // the batch's rows are contiguous in the cache
            return linear_desc(x, d.b * d.sk, w, bias, dst, e);
        SgemmDesc g;  // one slice per batch, the weight shared (batch_b = 1)
        g.trans_b = true;
        g.m = d.sk;
        g.n = e;
        g.k = e;
        g.a = x;
        g.lda = e;
        g.stride_a = d.sk * e;
        g.batch_a = d.b;
        g.b = w;
        g.ldb = e;
        g.c = dst;
        g.ldc = e;
        g.stride_c = d.capacity * e;
        g.batch = d.b;
        g.bias = bias;
        return g;
    };

    const SgemmDesc proj[3] = {linear_desc(d.query, d.b * d.sq, d.wq, d.bq, qbuf, e),
                               cache_desc(d.key, d.wk, d.bk, d.k_cache), cache_desc(d.value, d.wv, d.bv, d.v_cache)};
    const int nproj = d.sk > 0 ? 3 : 1;
    // Up to 64 rows (the same rows of query, key and value) the three
    // projections share one launch: 3x the columns fill the GPU better than
    // one projection does, and two launch tails go away.
    if (sgemm_nt_group_fits(proj, nproj)) {
        GFH_TRY(launch_sgemm_nt_group(proj, nproj, s));
    } else {
        for (int i = 0; i < nproj; ++i) GFH_TRY(launch_sgemm(proj[i], s));
    }
    const int64_t kv_len = d.past_len + d.sk;
    if (d.sq <= 16) {
        KvAttnDesc a;
        a.q = qbuf;
        a.k = d.k_cache;
        a.v = d.v_cache;
        a.out = abuf;
        a.weights = d.weights;
        a.mask = d.mask;
        a.mask_numel = d.mask_numel;
        a.q_bs = d.sq * e;
        a.q_rs = e;
        a.kv_bs = d.capacity * e;
        a.kv_rs = e;
        a.o_bs = d.sq * e;
        a.o_rs = e;
        a.b = d.b;
        a.h = d.h;
        a.sq = d.sq;
        a.kv_len = kv_len;
        a.d = hd;
        a.scale = d.scale;
        a.causal = d.causal;
        GFH_TRY(launch_kv_attention(a, s));
    } else {
        SdpaDesc a;
        a.q = qbuf;
        a.k = d.k_cache;
        a.v = d.v_cache;
        a.out = abuf;
        a.weights = d.weights;
        a.b = d.b;
        a.h = d.h;
        a.sq = d.sq;
        a.skv = kv_len;
        a.d = hd;
        a.scale = d.scale;
        a.causal = d.causal;
        a.mask = d.mask;
        a.mask_numel = d.mask_numel;
        a.strided = true;
        a.q_bs = d.sq * e, a.q_hs = hd, a.q_rs = e;
        a.kv_bs = d.capacity * e, a.kv_hs = hd, a.kv_rs = e;
        a.o_bs = d.sq * e, a.o_hs = hd, a.o_rs = e;
        GFH_TRY(launch_sdpa(a, s));
    }
    return launch_sgemm(linear_desc(abuf, d.b * d.sq, d.wo, d.bo, d.out, e), s);
}

}  // namespace gfh
