// gemm_nt_skinny.hip -- Linear::forward for a few rows of x:
// y = alpha * x . W^T (+ beta y) (+ bias), x [m, k] with 4 < m <= 64 and W
// [n, k] row-major, the reference's [out, in] weight
// (ghostflow-nn/src/linear.rs:56-69) as gfh_sgemm's NT form.
//
// At these sizes the layer is HBM-bound up to m ~ 40 (every weight byte is
// used m times) and no tile GEMM fills the GPU: a 64-row tile wastes most
// of its MFMA rows and a grid of n / 64 workgroups cannot stream W.  So the
// weight is streamed from HBM straight into v_mfma_f32_16x16x4_f32
// operands:
//  * a workgroup owns 64 weight rows (output columns) over one K-slice;
//    wave w owns rows 16 w .. 16 w + 15 and computes all m rows of x for
//    them, so no sums cross waves;
//  * K advances in chunks of 64 elements (256 bytes of every row).  Lane l
//    holds 16 bytes of weight row l % 16 at element 16 s + 4 (l / 16) of
//    step s of the chunk, and the same elements of x row l % 16 (+ 16 per
//    row block); element e of those vectors feeds MFMA e, so the four MFMAs
//    of a step pair every (row, k) of x with the same k of W;
//  * the chunk of x is staged once per workgroup and read by all four
//    waves: a 3-stage LDS ring filled by global_load_lds_dwordx4 (1 KB per
//    instruction: 4 rows x 256 bytes), 16-byte slots swizzled by row so the
//    fragment reads are conflict-free.  Read per wave straight from L2 (as
//    the weight is), x made every workgroup move m / 16 times the weight
//    bytes again: a read-only probe of the weight stream at [4096, 4096]
//    took 12.8 us alone and 18.2 us with the x reads of m = 16;
//  * the weight chunks go through an LDS ring of their own, two chunks ahead
//    of the MFMAs: each wave fills its 16 rows with global_load_lds_dwordx4,
//    4 rows x 256 bytes (whole 128-byte lines) per instruction, swizzled as
//    x is, and reads its MFMA fragments back with ds_read_b128.  Loaded
//    straight into the fragments' registers, one instruction covered 16
//    rows x 64 bytes (half lines); at [4096, 4096] the ring took 18.5 / 18.6
//    / 21.8 / 30.6 us at m = 8 / 16 / 32 / 64 against 19.2 / 19.2 / 22.7 /
//    34.3 us, the fp32 SwiGLU at m = 16 126.9 against 130.2 us, and three
//    chunks ahead were slower than two (18.8 against 18.5 us at m = 8);
//  * with fewer than ~512 workgroups K is also split over workgroups: each
//    wave publishes its partial block with agent-scope stores and counts
//    its arrival on its 16-column block, and the last one adds the slices
//    in slice order and runs the epilogue (alpha, + beta y, + bias:
//    separate f32 roundings, as in the tile GEMM).
// The sums are regrouped against the reference's sequential k order, so the
// result is within the fp32 GEMM bound (bit-exact when every partial sum is
// exact, e.g. on small-integer inputs).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace gfh {
namespace {

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(1))) void *glb_ptr;

constexpr int kWaves = 4;
constexpr int kGroupCols = 16 * kWaves;  // weight rows per workgroup
constexpr int kKC = 64;                  // k elements per chunk
constexpr int kRowBytes = kKC * 4;       // bytes of one row per chunk

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
    int64_t ngrp, kslice, slices;
    float *part;    // [groups][slices][m][n] partial sums (slices > 1, batch 1)
    int *counters;  // [groups][16-column blocks], zero at rest (slices > 1)
    // ngroups > 0: blockIdx.y selects product g of a grouped launch, with
    // the operands below (m, n, k, lda, ldb, alpha and beta are shared).
    int ngroups;
    const float *gx[kNtMaxGroups];
    const float *gw[kNtMaxGroups];
    float *gy[kNtMaxGroups];
    const float *gbias[kNtMaxGroups];
    int64_t gldc[kNtMaxGroups];
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// MB: 16-row blocks of x (m <= 16 MB); D: chunks in flight ahead of the
// MFMAs (D + 1 stages of each ring).  LDS: 12 KB x MB + 48 KB, so two
// workgroups per CU up to 32 rows and one above.
template <int MB, int D>
__global__ __launch_bounds__(64 * kWaves, MB <= 2 ? 2 : 1) void gemm_nt_skinny_kernel(SkNtParams p) {
    constexpr int kXRows = 16 * MB;
    constexpr int kStageBytes = kXRows * kRowBytes;
    constexpr int kWStageBytes = kGroupCols * kRowBytes;
    constexpr int kStages = D + 1;
    constexpr int kOps = MB + 4;  // vector memory instructions per chunk and wave
    __shared__ __attribute__((aligned(1024))) char xs[kStages * (kStageBytes + kWStageBytes)];
    char *const wsm = xs + kStages * kStageBytes;  // the weight ring
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t grp = blockIdx.x % p.ngrp, slice = blockIdx.x / p.ngrp;
    const int64_t n0 = grp * kGroupCols + 16 * wave;  // this wave's first weight row
    // blockIdx.y: product z of a grouped launch, else batch slice z with the
    // reference's modulo indexing (matmul.rs:147-149)
    const uint32_t z = blockIdx.y;
    const bool grouped = p.ngroups > 0;
    const float *xb = grouped ? p.gx[z] : p.x + (int64_t)(z % (uint32_t)p.batch_a) * p.stride_a;
    const float *wb = grouped ? p.gw[z] : p.w + (int64_t)(z % (uint32_t)p.batch_b) * p.stride_b;
    float *yb = grouped ? p.gy[z] : p.y + (int64_t)z * p.stride_c;
    const float *bias = grouped ? p.gbias[z] : p.bias;
    const int64_t ldc = grouped ? p.gldc[z] : p.ldc;
    // (split-K buffers exist only when K is split)
    float *part = grouped && p.part ? p.part + (int64_t)z * p.slices * p.m * p.n : p.part;
    int *counters = grouped && p.counters ? p.counters + (int64_t)z * p.ngrp * kWaves : p.counters;

    const int64_t k_lo = slice * p.kslice;
    const int kl = (int)min(p.kslice, p.k - k_lo);  // > 0, a multiple of 4
    const int nch = (kl + kKC - 1) / kKC;

    // x: instruction j of wave w fills stage rows 4 (w MB + j) .. + 3; lane l
    // fills slot l % 16 of row l / 16 of them from logical 16-byte chunk
    // (l % 16) ^ (row % 16).  Rows past m read row m - 1 (never stored);
    // elements past the slice read its last four (masked in the tail).
    const float *xsrc[MB];
    int xcol[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        const int r = 4 * (wave * MB + j) + (lane >> 4);
        xsrc[j] = xb + min<int64_t>(r, p.m - 1) * p.lda + k_lo;
        xcol[j] = 4 * ((lane & 15) ^ (r & 15));
    }
    auto issue_x = [&](int i, int slot) __attribute__((always_inline)) {
        char *stage = xs + slot * kStageBytes;
#pragma unroll
        for (int j = 0; j < MB; ++j)
            __builtin_amdgcn_global_load_lds((glb_ptr)(xsrc[j] + min(i * kKC + xcol[j], kl - 4)),
                                             (lds_ptr)(stage + 4 * (wave * MB + j) * kRowBytes), 16, 0, 0);
    };
    // W: instruction j of wave w fills its rows 4 j .. 4 j + 3 of the stage;
    // lane l fills slot l % 16 of row 4 j + l / 16 from logical chunk
    // (l % 16) ^ row, the swizzle of the x ring.  Rows past n read row n - 1
    // (never stored); elements past the slice read its last four (masked in
    // the tail).
    const float *wrow[4];
    int wcol[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + (lane >> 4);
        wrow[j] = wb + min<int64_t>(n0 + r, p.n - 1) * p.ldb + k_lo;
        wcol[j] = 4 * ((lane & 15) ^ r);
    }
    auto issue_w = [&](int i, int slot) __attribute__((always_inline)) {
        char *stage = wsm + slot * kWStageBytes + wave * 16 * kRowBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_global_load_lds((glb_ptr)(wrow[j] + min(i * kKC + wcol[j], kl - 4)),
                                             (lds_ptr)(stage + 4 * j * kRowBytes), 16, 0, kNtHint);
    };

    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Fragment of x block mb, step s: row 16 mb + l % 16, logical chunk
    // 4 s + l / 16 (block rows start at multiples of 16, so the swizzle is
    // the lane's own l % 16); the weight fragment is the same slot of row
    // l % 16 of the wave's rows in the weight stage.
    const int xrd = (lane & 15) * kRowBytes;
    const int lane_sw = lane & 15;
    const int kq = 4 * (lane >> 4);  // the lane's k offset within a step
    auto compute = [&](int u, auto tail, int i) __attribute__((always_inline)) {
        const char *stage = xs + u * kStageBytes;
        const char *wstage = wsm + u * kWStageBytes + wave * 16 * kRowBytes + xrd;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            f32x4 xv[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                xv[mb] = *reinterpret_cast<const f32x4 *>(stage + mb * 16 * kRowBytes + xrd +
                                                          (((4 * s + (lane >> 4)) ^ (lane & 15)) << 4));
            f32x4 wv = *reinterpret_cast<const f32x4 *>(wstage + (((4 * s + (lane >> 4)) ^ lane_sw) << 4));
            if constexpr (decltype(tail)::value) {
                // k % 4 == 0: a lane's 4 elements are all inside the slice or
                // all past it; past it both operands are zero (a zero x alone
                // would turn an inf weight into NaN).
                const bool ok = i * kKC + 16 * s + kq < kl;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    wv[e] = ok ? wv[e] : 0.f;
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) xv[mb][e] = ok ? xv[mb][e] : 0.f;
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[mb][e], wv[e], acc[mb], 0, 0, 0);
        }
    };

    // Chunk i (ring stage u = i % kStages): wait for its x and W (the next
    // D - 1 chunks' loads stay in flight), barrier (its x is visible, and
    // every wave is done with chunk i - 1, whose stages now refill), issue
    // chunk i + D, compute chunk i.  The issue is unconditional -- past the
    // last chunk it repeats the last one (an L2 hit) into the free stages --
    // so every chunk issues the same kOps instructions per wave, in the same
    // order, and the wait count is a constant.
    const bool ragged = (kl % kKC) != 0;
    auto step = [&](int i, int u) __attribute__((always_inline)) {
        static_assert(D >= 1 && (D - 1) * kOps < 64, "the wait count must fit vmcnt");
        wait_vmcnt<(D - 1) * kOps>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int nx = min(i + D, nch - 1);
        issue_x(nx, (u + D) % kStages);
        __builtin_amdgcn_sched_barrier(0);
        issue_w(nx, (u + D) % kStages);
        __builtin_amdgcn_sched_barrier(0);
        if (ragged && i + 1 == nch)
            compute(u, std::true_type{}, i);
        else
            compute(u, std::false_type{}, i);
    };
#pragma unroll
    for (int c = 0; c < D; ++c) {
        issue_x(min(c, nch - 1), c);
        __builtin_amdgcn_sched_barrier(0);
        issue_w(min(c, nch - 1), c);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Whole rounds of kStages chunks (stage indices known at compile time),
    // then the chunks left.
    int i = 0;
    for (; i + kStages <= nch; i += kStages) {
#pragma unroll
        for (int u = 0; u < kStages; ++u) step(i + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < kStages; ++u)
        if (i + u < nch) step(i + u, u);
    wait_vmcnt<0>();  // no load may still be writing the ring
    if (n0 >= p.n) return;  // a wave past the last column (after every barrier)

    // 16x16 accumulator layout: lane l, register r -> row 4 (l / 16) + r of
    // the block, column l % 16.
    const int64_t col = n0 + (lane & 15);
    auto row_of = [&](int mb, int r) -> int64_t { return (int64_t)mb * 16 + 4 * (lane >> 4) + r; };
    auto epilogue = [&](int64_t row, float sum) {
        float *dst = yb + row * ldc + col;
        float v = p.alpha * sum;
        if (p.beta != 0.f) v = v + p.beta * *dst;
        if (bias) v = v + bias[col];
        *dst = v;
    };
    const bool col_ok = col < p.n;

    if (p.slices == 1) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_of(mb, r);
                if (row < p.m && col_ok) epilogue(row, acc[mb][r]);
            }
        return;
    }

    // Publish the partial block with agent-scope stores (they reach the
    // device coherence point, so no cache writeback is needed), wait for
    // them, then count this wave's arrival on its column block.
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = row_of(mb, r);
            if (row < p.m && col_ok)
                __hip_atomic_store(part + (slice * p.m + row) * p.n + col, acc[mb][r], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    // split-K arrival protocol (common.hpp): steps 2-4
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    wait_vmcnt<0>();
    const int64_t blk = n0 / 16;
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(counters + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (int)p.slices - 1;
    last = __shfl(last, 0);
    if (!last) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // The lane requests the partials of all its outputs for kGroup slices
    // at a time before adding any of them, so the loads overlap instead of
    // paying one memory latency per output and slice; each output is still
    // summed in slice order.
    constexpr int kGroup = 32 / (4 * MB) > 0 ? 32 / (4 * MB) : 1;
    const float *src[MB][4];
    float sum[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = row_of(mb, r);
            src[mb][r] = (row < p.m && col_ok) ? part + row * p.n + col : nullptr;
            sum[mb][r] = 0.f;
        }
    for (int64_t j0 = 0; j0 < p.slices; j0 += kGroup) {
        float pv[kGroup][MB][4];
#pragma unroll
        for (int g = 0; g < kGroup; ++g)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    pv[g][mb][r] = (src[mb][r] && j0 + g < p.slices)
                                       ? __hip_atomic_load(src[mb][r] + (j0 + g) * p.m * p.n, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                       : 0.f;
#pragma unroll
        for (int g = 0; g < kGroup; ++g)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (j0 + g < p.slices) sum[mb][r] = (j0 + g == 0) ? pv[g][mb][r] : sum[mb][r] + pv[g][mb][r];
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (src[mb][r]) epilogue(row_of(mb, r), sum[mb][r]);
    if (lane == 0) __hip_atomic_store(counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K elements per workgroup: all of K with at least ~kTargetWgs workgroups
// (or a batched call), otherwise enough slices for about that many, each at
// least 4 chunks, a multiple of the chunk.  At [4096, 4096] (64 column
// groups): 8 slices took 18.8 / 18.7 / 22.2 / 34.3 us at m = 8 / 16 / 32 /
// 64, against 20.4-22.9 / 21.8-25.4 / 29-34 us with 4 and 21.3 / 27.2 /
// 41.7 us (m = 8 / 32 / 64) with 16.  Of the 18.7 us at m = 16, about 2.7
// us are the split-K tail (partial stores, arrival count, the last
// arriver's reads: three memory round trips) and 1 us the x staging.
// Above 32 rows (three or four row blocks: one workgroup per CU, its LDS
// rings 84-96 KB) half as many workgroups, one round of them: m = 40 / 48 /
// 64 took 25.7 / 25.6 / 30.6 us against 28.5 / 28.9 / 34.3 us with the
// weights in registers and 512 workgroups for m <= 48, while m <= 32
// prefers 8 slices.
constexpr int64_t kTargetWgs = 512;
constexpr int kDepth = 2;
// Up to 32 rows the slice count is rounded down: at N = 11008 (172 groups),
// K = 4096, 2 slices took 45.9 / 46.8 / 56.8 us at m = 8 / 16 / 32 against
// 49.9 / 50.3 / 57.4 with 3 (uneven: 1536, 1536, 1024 rows) and 57.6 /
// 57.8 / 68.3 with none.
int64_t choose_kslice(int64_t ngrp, int64_t k, int64_t batch, int64_t m) {
    const int64_t kc = ((k + kKC - 1) / kKC) * kKC;
    if (batch > 1) return kc;
    int64_t s = m > 32 ? (kTargetWgs / 2 + ngrp - 1) / ngrp : kTargetWgs / ngrp;
    s = std::max<int64_t>(1, std::min<int64_t>(s, k / (4 * kKC)));
    const int64_t ks = (k + s - 1) / s;
    return (ks + kKC - 1) / kKC * kKC;
}

}  // namespace

bool gemm_nt_skinny_fits(const SgemmDesc &d) {
    return !d.trans_a && d.trans_b && d.m > kNtSkinnyMinM && d.m <= 64 && d.k > 0 && d.n > 0 && d.k % 4 == 0 &&
           d.lda % 4 == 0 && d.ldb % 4 == 0 && aligned16(d.a) && aligned16(d.b) &&
           (d.batch_a <= 1 || d.stride_a % 4 == 0) && (d.batch_b <= 1 || d.stride_b % 4 == 0) && d.batch <= 65535;
}

namespace {
// Slicing, split-K buffers and the launch for `gy` products (grid.y).
int launch_params(SkNtParams &p, int64_t gy, hipStream_t s) {
    const int64_t prods = p.ngroups > 0 ? p.ngroups : 1;
    p.ngrp = (p.n + kGroupCols - 1) / kGroupCols;
    p.kslice = choose_kslice(p.ngrp * prods, p.k, p.ngroups > 0 ? 1 : gy, p.m);
    p.slices = (p.k + p.kslice - 1) / p.kslice;
    if (p.slices > 1) {
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(float) * (size_t)(prods * p.slices * p.m * p.n), &ws));
        p.part = static_cast<float *>(ws);
        GFH_TRY(stream_counters(s, (size_t)(prods * p.ngrp * kWaves), &p.counters));
    }
    const dim3 grid((unsigned)(p.ngrp * p.slices), (unsigned)gy), block(64 * kWaves);
    if (p.m <= 16)
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<1, kDepth>), grid, block, 0, s, p);
    else if (p.m <= 32)
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<2, kDepth>), grid, block, 0, s, p);
    else if (p.m <= 48)
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<3, kDepth>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((gemm_nt_skinny_kernel<4, kDepth>), grid, block, 0, s, p);
    return check_launch("sgemm (NT skinny MFMA)");
}
}  // namespace

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
    return launch_params(p, std::max<int64_t>(d.batch, 1), s);
}

bool gemm_nt_skinny_group_fits(const SgemmDesc *d, int count) {
    if (count < 1 || count > kNtMaxGroups) return false;
    for (int g = 0; g < count; ++g) {
        const SgemmDesc &e = d[g];
        if (!gemm_nt_skinny_fits(e) || e.batch > 1 || e.m != d[0].m || e.n != d[0].n || e.k != d[0].k ||
            e.lda != d[0].lda || e.ldb != d[0].ldb || e.alpha != d[0].alpha || e.beta != d[0].beta)
            return false;
    }
    return true;
}

int launch_gemm_nt_skinny_group(const SgemmDesc *d, int count, hipStream_t s) {
    SkNtParams p{};
    p.lda = d[0].lda;
    p.ldb = d[0].ldb;
    p.batch_a = p.batch_b = 1;
    p.m = d[0].m;
    p.n = d[0].n;
    p.k = d[0].k;
    p.alpha = d[0].alpha;
    p.beta = d[0].beta;
    p.ngroups = count;
    for (int g = 0; g < count; ++g) {
        p.gx[g] = d[g].a;
        p.gw[g] = d[g].b;
        p.gy[g] = d[g].c;
        p.gbias[g] = d[g].bias;
        p.gldc[g] = d[g].ldc;
    }
    return launch_params(p, count, s);
}

}  // namespace gfh
