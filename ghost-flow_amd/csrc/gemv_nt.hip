// gemv_nt.hip -- Linear::forward at decode sizes: y = alpha * x . W^T (+ beta y)
// (+ bias) with x [m <= 4, k] and W [n, k] row-major, the reference's
// [out, in] weight (ghostflow-nn/src/linear.rs:56-69).  HBM-bound: every
// weight byte is read once, and the m rows of x are re-read from L2.
//
// A weight row is contiguous in k, so the natural split is the row dot
// product: lanes stride over k in 16-byte pieces (lane l takes k = 4l + 256t),
// each load instruction reading 1 KB of one row, and the R x m partial sums
// of a lane are added over the wave with DPP at the end.  A workgroup owns R
// rows and its 4 waves take every 4th 256-element step of them, so a wave
// re-reads only its quarter of x for all R rows; the 4 wave totals are added
// in LDS in a fixed order.  The sums are regrouped against the reference's
// sequential k order, so the result is within the fp32 GEMM bound, not
// bit-identical.
//
// gfh_sgemm sends an NT call here when m <= 4 and the operands allow 16-byte
// loads (k, lda, ldb multiples of 4; 16-byte aligned A and B); batched calls
// keep the reference's modulo batch indexing (matmul.rs:147-149).  A grouped
// launch runs up to kNtMaxGroups such products of one shape, each with its
// own x, W, y, bias and ldc (the q / k / v projections of a
// MultiHeadAttention decode step, attention.rs:108-114).
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

// Every f32 product and sum is its own rounding, as in the reference CPU
// path (no FMA contraction).
#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kNtWaves = 4;

struct NtParams {
    const float *x;  // [batch_a][m][lda]
    const float *w;  // [batch_b][n][ldb]
    float *y;        // [batch][m][ldc]
    const float *bias;
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;
    int64_t batch_a, batch_b;
    int64_t m, n, k;
    float alpha, beta;
    // ngroups > 0: blockIdx.y selects product g of a grouped launch, with
    // the operands below (m, n, k, lda, ldb, alpha and beta are shared).
    int ngroups;
    const float *gx[kNtMaxGroups];
    const float *gw[kNtMaxGroups];
    float *gy[kNtMaxGroups];
    const float *gbias[kNtMaxGroups];
    int64_t gldc[kNtMaxGroups];
};

// The operands of one workgroup's product.
struct NtSlice {
    const float *x, *w;
    float *y;
    const float *bias;
    int64_t ldc;
};

// Operands of blockIdx.y: group g of a grouped launch, else batch slice z
// with the reference's modulo indexing.  Batch counts are below 2^16, so
// 32-bit arithmetic suffices (a 64-bit remainder expands to a long
// instruction sequence), and a single slice skips it.
__device__ __forceinline__ NtSlice slice_of(const NtParams &p) {
    const uint32_t z = blockIdx.y;
    if (p.ngroups > 0) return {p.gx[z], p.gw[z], p.gy[z], p.gbias[z], p.gldc[z]};
    if (z == 0) return {p.x, p.w, p.y, p.bias, p.ldc};
    return {p.x + (int64_t)(z % (uint32_t)p.batch_a) * p.stride_a, p.w + (int64_t)(z % (uint32_t)p.batch_b) * p.stride_b,
            p.y + (int64_t)z * p.stride_c, p.bias, p.ldc};
}

// Same contract, K split over the workgroup's waves: wave w takes the
// 256-element steps t = w, w + 4, ... of the workgroup's R rows (the partial
// last step, if any, belongs to the wave whose turn it is).
template <int MB, int R, int U>
__global__ __launch_bounds__(64 * kNtWaves, 2) void gemv_nt_ksplit_kernel(NtParams p) {
    __shared__ float red[kNtWaves][R * MB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n0 = (int64_t)blockIdx.x * R;
    const NtSlice sl = slice_of(p);

    const float *wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r] = sl.w + std::min<int64_t>(n0 + r, p.n - 1) * p.ldb + 4 * lane;
    const float *xr[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) xr[b] = sl.x + std::min<int64_t>(b, p.m - 1) * p.lda + 4 * lane;

    float acc[R][MB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[r][b] = 0.f;
    auto fma4 = [&](const f32x4 (&wv)[R], const f32x4 (&xv)[MB]) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[r][b] = fmaf(wv[r][e], xv[b][e], acc[r][b]);
    };

    const int64_t full = p.k / 256;
    int64_t t = wave;
    for (; t + kNtWaves * (U - 1) < full; t += kNtWaves * U) {
        f32x4 wv[U][R], xv[U][MB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                wv[u][r] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(wr[r] + (t + kNtWaves * u) * 256));
#pragma unroll
            for (int b = 0; b < MB; ++b)
                xv[u][b] = *reinterpret_cast<const f32x4 *>(xr[b] + (t + kNtWaves * u) * 256);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) fma4(wv[u], xv[u]);
    }
    for (; t < full; t += kNtWaves) {
        f32x4 wv[R], xv[MB];
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(wr[r] + t * 256));
#pragma unroll
        for (int b = 0; b < MB; ++b) xv[b] = *reinterpret_cast<const f32x4 *>(xr[b] + t * 256);
        fma4(wv, xv);
    }
    if (full * 256 < p.k && t == full) {  // the partial step is this wave's turn (wave-uniform)
        const bool in = full * 256 + 4 * lane < p.k;
        const int64_t off = in ? full * 256 : -4 * (int64_t)lane;
        const uint32_t keep = in ? 0xffffffffu : 0u;
        f32x4 wv[R], xv[MB];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(wr[r] + off));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ve = v[e];  // (a bit cast of the element lvalue would read element 0)
                wv[r][e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, ve) & keep);
            }
        }
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(xr[b] + off);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ve = v[e];
                xv[b][e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, ve) & keep);
            }
        }
        fma4(wv, xv);
    }

    // All the wave sums first, then the stores: a store under a lane
    // condition between them would serialize the reductions.
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[r][b] = wave_sum(acc[r][b]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < MB; ++b) red[wave][r * MB + b] = acc[r][b];
    }
    __syncthreads();
    const int idx = threadIdx.x;
    if (idx < R * MB) {
        const int r = idx / MB, b = idx % MB;
        const int64_t col = n0 + r;
        if (col < p.n && b < p.m) {
            float *dst = sl.y + b * sl.ldc + col;
            float v = p.alpha * ((red[0][idx] + red[1][idx]) + (red[2][idx] + red[3][idx]));
            if (p.beta != 0.f) v = v + p.beta * *dst;
            if (sl.bias) v = v + sl.bias[col];
            *dst = v;
        }
    }
}

// 2 rows per workgroup up to 2 rows of x, 4 rows at 3-4 (x re-read from L2
// at most twice the weight bytes).  Measured on [4096, 4096] / [12288, 4096]:
// m = 1 12.8 / 33.1 us, m = 4 15.2 / 38.4 us, against 13.4 / 35.1 and
// 16.9 / 43.3 us with one row group per wave.  grid.y: batch slices or groups.
template <int MB>
int launch_mb(const NtParams &p, int64_t gy, hipStream_t s) {
    constexpr int R = MB <= 2 ? 2 : 4;
    constexpr int U = MB <= 2 ? 2 : 1;
    const dim3 grid((unsigned)((p.n + R - 1) / R), (unsigned)gy), block(64 * kNtWaves);
    hipLaunchKernelGGL((gemv_nt_ksplit_kernel<MB, R, U>), grid, block, 0, s, p);
    return check_launch("sgemm (NT GEMV)");
}

int launch_m(const NtParams &p, int64_t gy, hipStream_t s) {
    if (p.m == 1) return launch_mb<1>(p, gy, s);
    if (p.m == 2) return launch_mb<2>(p, gy, s);
    return launch_mb<4>(p, gy, s);
}

}  // namespace

bool gemv_nt_fits(const SgemmDesc &d) {
    return !d.trans_a && d.trans_b && d.m >= 1 && d.m <= kNtSkinnyMinM && d.k > 0 && d.n > 0 && d.k % 4 == 0 &&
           d.lda % 4 == 0 && d.ldb % 4 == 0 && aligned16(d.a) && aligned16(d.b) &&
           (d.batch_a <= 1 || d.stride_a % 4 == 0) && (d.batch_b <= 1 || d.stride_b % 4 == 0) && d.batch <= 65535;
}

int launch_gemv_nt(const SgemmDesc &d, hipStream_t s) {
    NtParams p{};
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
    return launch_m(p, std::max<int64_t>(d.batch, 1), s);
}

bool gemv_nt_group_fits(const SgemmDesc *d, int count) {
    if (count < 1 || count > kNtMaxGroups) return false;
    for (int g = 0; g < count; ++g) {
        const SgemmDesc &e = d[g];
        if (!gemv_nt_fits(e) || e.batch > 1 || e.m != d[0].m || e.n != d[0].n || e.k != d[0].k ||
            e.lda != d[0].lda || e.ldb != d[0].ldb || e.alpha != d[0].alpha || e.beta != d[0].beta)
            return false;
    }
    return true;
}

int launch_gemv_nt_group(const SgemmDesc *d, int count, hipStream_t s) {
    NtParams p{};
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
    return launch_m(p, count, s);
}

}  // namespace gfh
