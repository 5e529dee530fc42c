// gemm_nt_skinny.hip -- Linear::forward for a few rows of x:
// y = alpha * x . W^T (+ beta y) (+ bias), x [m, k] with 4 < m <= 64 and W
// [n, k] row-major, the reference's [out, in] weight
// (ghostflow-nn/src/linear.rs:56-69) as gfh_sgemm's NT form.
//
// At these sizes the layer is HBM-bound up to m ~ 40 (every weight byte is
// used m times) and no tile GEMM fills the GPU: a 64-row tile wastes most
// of its MFMA rows and a grid of n / 64 workgroups cannot stream W.  So the
// weight is streamed from HBM straight into v_mfma_f32_16x16x4_f32 operands,
// as the skinny int8 linear does:
//  * a workgroup owns NB blocks of 16 output columns (weight rows); lane l
//    reads 16 bytes of row l % 16 of each block at float offset 4 * (l / 16)
//    of each 16-float k-step, and the same bytes of x row l % 16 (+ 16 per
//    row block); element e of those vectors feeds MFMA e, so the four MFMAs
//    of a step pair every (row, k) of x with the same k of W.  NB = 1: at
//    [4096, 4096] two or four blocks per workgroup (x re-read half or a
//    quarter as often) measured slower, 30.9 against 27.4 us at m = 16 and
//    93 against 67 us at m = 64, as the grid shrinks by the same factor;
//  * the 4 waves take contiguous quarters of the workgroup's k-steps and
//    their accumulators are added in LDS in a fixed order;
//  * with fewer than ~512 column blocks K is also split over workgroups:
//    each publishes its partial tile with agent-scope stores and counts its
//    arrival, and the last one adds the slices in slice order and runs the
//    epilogue (alpha, + beta y, + bias: separate f32 roundings, as in the
//    tile GEMM).
// The sums are regrouped against the reference's sequential k order, so the
// result is within the fp32 GEMM bound (bit-exact when every partial sum is
// exact, e.g. on small-integer inputs).
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kWaves = 4;

struct SkNtParams {
    const float *x;  // [batch_a][m][lda]
    const float *w;  // [batch_b][n][ldb]
    float *y;        // [batch][m][ldc]
    const float *bias;
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;
    int64_t batch_a, batch_b;
    int64_t m, n, k;
    float alpha, beta;
    int64_t nblk, kslice, slices;
    float *part;    // [slices][m][n] partial sums (slices > 1, batch 1)
    int *counters;  // one per column block, zero at rest (slices > 1)
};

// MB: 16-row blocks of x (m <= 16 MB); NB: 16-column blocks per workgroup.
template <int MB, int NB>
__global__ __launch_bounds__(64 * kWaves) void gemm_nt_skinny_kernel(SkNtParams p) {
    constexpr int kU = MB * NB > 2 ? 4 : 8;  // k-steps in flight per lane
    __shared__ f32x4 red[kWaves - 1][MB * NB][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t blk = blockIdx.x % p.nblk, slice = blockIdx.x / p.nblk;
    const int64_t n0 = blk * 16 * NB;
    // batch slice blockIdx.y with the reference's modulo indexing
    // (matmul.rs:147-149)
    const uint32_t z = blockIdx.y;
    const float *xb = p.x + (int64_t)(z % (uint32_t)p.batch_a) * p.stride_a;
    const float *wb = p.w + (int64_t)(z % (uint32_t)p.batch_b) * p.stride_b;
    float *yb = p.y + (int64_t)z * p.stride_c;

    const int64_t k_lo = slice * p.kslice;
    const int kl = (int)min(p.kslice, p.k - k_lo);  // a multiple of 4
    const int nsteps = (kl + 15) / 16;
    const int per = (nsteps + kWaves - 1) / kWaves;
    const int st0 = min(wave * per, nsteps), st1 = min(st0 + per, nsteps);

    // Rows past n read row n - 1 and rows past m read row m - 1: their sums
    // are never stored, and the loads need no condition.
    const int kq = 4 * (lane >> 4);
    const float *wsrc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) wsrc[nb] = wb + min(n0 + nb * 16 + (lane & 15), p.n - 1) * p.ldb + k_lo + kq;
    const float *xsrc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xsrc[mb] = xb + min<int64_t>(mb * 16 + (lane & 15), p.m - 1) * p.lda + k_lo + kq;

    f32x4 acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = st0; s0 < st1; s0 += kU) {
        f32x4 wv[kU][NB], xv[kU][MB];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            // k % 4 == 0: a lane's 4 floats are all inside the slice or all
            // past it; past it both operands are zero (a zero x alone would
            // turn an inf weight into NaN).
            const int off = (s0 + u) * 16;
            const bool ok = s0 + u < st1 && off + kq < kl;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                wv[u][nb] = ok ? *reinterpret_cast<const f32x4 *>(wsrc[nb] + off) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                xv[u][mb] = ok ? *reinterpret_cast<const f32x4 *>(xsrc[mb] + off) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const float xe = xv[u][mb][e];
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        const float we = wv[u][nb][e];
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xe, we, acc[mb][nb], 0, 0, 0);
                    }
                }
    }

    // The four waves' partial sums, added in wave order in wave 0.
    if (wave > 0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) red[wave - 1][mb * NB + nb][lane] = acc[mb][nb];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int w2 = 0; w2 < kWaves - 1; ++w2) acc[mb][nb] = acc[mb][nb] + red[w2][mb * NB + nb][lane];

    // 16x16 accumulator layout: lane l, register r -> row 4 * (l / 16) + r,
    // column l % 16 of the block.
    auto col_of = [&](int nb) -> int64_t { return n0 + nb * 16 + (lane & 15); };
    auto row_of = [&](int mb, int r) -> int64_t { return (int64_t)mb * 16 + 4 * (lane >> 4) + r; };
    auto epilogue = [&](int64_t row, int64_t col, float sum) {
        float *dst = yb + row * p.ldc + col;
        float v = p.alpha * sum;
        if (p.beta != 0.f) v = v + p.beta * *dst;
        if (p.bias) v = v + p.bias[col];
        *dst = v;
    };

    if (p.slices == 1) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = row_of(mb, r), col = col_of(nb);
                    if (row < p.m && col < p.n) epilogue(row, col, acc[mb][nb][r]);
                }
        return;
    }

    // Publish the partial tile with agent-scope stores (they reach the
    // device coherence point, so no cache writeback is needed), wait for
    // them, then count this workgroup's arrival.
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_of(mb, r), col = col_of(nb);
                if (row < p.m && col < p.n)
                    __hip_atomic_store(p.part + (slice * p.m + row) * p.n + col, acc[mb][nb][r], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(p.counters + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (int)p.slices - 1;
    last = __shfl(last, 0);
    if (!last) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_of(mb, r), col = col_of(nb);
                if (row >= p.m || col >= p.n) continue;
                const float *src = p.part + row * p.n + col;
                float sum = 0.f;
                for (int64_t j = 0; j < p.slices; ++j)
                    sum = sum + __hip_atomic_load(src + j * p.m * p.n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                epilogue(row, col, sum);
            }
    if (lane == 0) __hip_atomic_store(p.counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K elements per workgroup: all of K with at least ~512 column blocks (or a
// batched call), otherwise enough slices for ~512 workgroups, each at least
// 1024 elements, a multiple of 16.
int64_t choose_kslice(int64_t nblk, int64_t k, int64_t batch) {
    if (batch > 1) return k;
    int64_t s = (512 + nblk - 1) / nblk;
    s = std::max<int64_t>(1, std::min<int64_t>(s, k / 1024));
    const int64_t ks = (k + s - 1) / s;
    return (ks + 15) & ~(int64_t)15;
}

}  // namespace

bool gemm_nt_skinny_fits(const SgemmDesc &d) {
    return !d.trans_a && d.trans_b && d.m > kNtSkinnyMinM && d.m <= 64 && d.k > 0 && d.n > 0 && d.k % 4 == 0 &&
           d.lda % 4 == 0 && d.ldb % 4 == 0 && aligned16(d.a) && aligned16(d.b) &&
           (d.batch_a <= 1 || d.stride_a % 4 == 0) && (d.batch_b <= 1 || d.stride_b % 4 == 0) && d.batch <= 65535;
}

int launch_gemm_nt_skinny(const SgemmDesc &d, hipStream_t s) {
    SkNtParams p{};
    p.x = d.a;
    p.w = d.b;
    p.y = d.c;
    p.bias = d.bias;
    p.lda = d.lda;
    p.ldb = d.ldb;
    p.ldc = d.ldc;
    p.stride_a = d.stride_a;
    p.stride_b = d.stride_b;
    p.stride_c = d.stride_c;
    p.batch_a = std::max<int64_t>(d.batch_a, 1);
    p.batch_b = std::max<int64_t>(d.batch_b, 1);
    p.m = d.m;
    p.n = d.n;
    p.k = d.k;
    p.alpha = d.alpha;
    p.beta = d.beta;
    const int64_t batch = std::max<int64_t>(d.batch, 1);
    constexpr int NB = 1;
    p.nblk = (d.n + 16 * NB - 1) / (16 * NB);
    p.kslice = choose_kslice(p.nblk, d.k, batch);
    p.slices = (d.k + p.kslice - 1) / p.kslice;
    if (p.slices > 1) {
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(float) * (size_t)(p.slices * d.m * d.n), &ws));
        p.part = static_cast<float *>(ws);
        GFH_TRY(stream_counters(s, (size_t)p.nblk, &p.counters));
    }
    const dim3 grid((unsigned)(p.nblk * p.slices), (unsigned)batch), block(64 * kWaves);
    if (d.m <= 16)
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<1, NB>), grid, block, 0, s, p);
    else if (d.m <= 32)
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<2, NB>), grid, block, 0, s, p);
    else if (d.m <= 48)
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<3, NB>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<4, NB>), grid, block, 0, s, p);
    return check_launch("sgemm (NT skinny MFMA)");
}

}  // namespace gfh
