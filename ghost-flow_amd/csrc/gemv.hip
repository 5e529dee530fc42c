// gemv.hip -- batched decode GEMV, HBM-bound: y[b,n] = sum_k x[b,k] * W[k,n]
// for W [K, N] row-major (Tensor::matmul with M = b,
// ghostflow-core/src/ops/matmul.rs:91-119), fp32 or int8 weights.
//
// The int8 form is DynamicQuantization::get_weights -> Tensor::matmul
// (ghostflow-nn/src/quantization.rs:173-204, :275-277) without ever
// materializing the fp32 weight:
//   y[b,n] = sum_k x[b,k] * ((q[k,n] - zp[k]) * s[k])
//          = sum_k xs[b,k] * q[k,n]  -  sum_k xs[b,k] * zp[k],   xs = x * s[k]
// so each weight costs one sign-extending convert and one FMA per batch row;
// the zero-point term is the same for every column and is subtracted once.
// (The products are regrouped, so the result is within the fp32 GEMM bound
// of the reference, not bit-identical to it.)
//
// Layout of the work (one kernel per call):
//  * A workgroup (4 wave64) owns a strip of 256 bytes of every W row (64
//    fp32 or 256 int8 columns) over one K-slice; lane l reads 16 bytes of
//    row (l / 16) of a 4-row group, so one load instruction covers 4 rows x
//    256 contiguous bytes and U of them per lane are in flight.  HBM streams
//    256-byte row runs at about 6 TB/s; 128-byte runs only reach ~5.
//  * Each wave walks a quarter of the slice; partial sums are reduced over
//    the 4 row lanes with xor shuffles, then over the 4 waves through LDS in
//    a fixed order.
//  * fp32 has 224 strips at N = 14336, enough workgroups to keep HBM busy,
//    so the slice is all of K and the workgroup writes y directly.  int8 has
//    only 56 strips, so K is split into S slices: every workgroup writes its
//    partial strip to a workspace, and the last of the S to finish (an
//    agent-scope arrival counter) adds the S partials in slice order and
//    writes y -- deterministic, one launch.  The counter is returned to 0
//    by that last workgroup.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace gfh {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kStripBytes = 256;

struct GemvParams {
    const float *x;
    const void *w;
    const float *scales;
    const int8_t *zps;
    float *y;
    float *part;    // [S][b][n] partial strips (S > 1)
    int *counters;  // one per strip, zero at rest (S > 1)
    int64_t b, k, n;
    int64_t nstrips;
    int64_t slices;
    int64_t kslice;  // rows per slice: a multiple of 16, at most kMaxSlice
};

constexpr int kMaxSlice = 1024;

template <typename WT, int MAXB, int U, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
    constexpr bool INT8 = sizeof(WT) == 1;
    constexpr int EPL = 16 / sizeof(WT);  // weights per lane per load
    constexpr int SCOLS = kStripBytes / sizeof(WT);
    // x of this slice's rows (int8: x * s[k]), [row][batch]
    __shared__ __attribute__((aligned(16))) float xs[kMaxSlice * MAXB];
    __shared__ float red[kWaves][MAXB][SCOLS];
    __shared__ float zred[kWaves][MAXB];
    __shared__ int last_flag;

    const WT *__restrict__ W = static_cast<const WT *>(p.w);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t strip = blockIdx.x % p.nstrips;
    const int64_t slice = blockIdx.x / p.nstrips;
    const int64_t col0 = strip * SCOLS;
    const int64_t col = col0 + (lane & 15) * EPL;
    const int rsub = lane >> 4;
    const int64_t nb = p.b < MAXB ? p.b : MAXB;
    const int64_t s_lo = slice * p.kslice;
    const int rows = (int)min(p.kslice, p.k - s_lo);

    float acc[MAXB][EPL];
#pragma unroll
    for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[bi][e] = 0.f;

    // Rows of this wave: a quarter of the slice, a multiple of 4.
    const int per = (((int)p.kslice + kWaves - 1) / kWaves + 3) & ~3;
    const int wb = min(wave * per, rows), we = min(wb + per, rows);
    const bool full_cols = VEC && (col + EPL - 1 < p.n);
    const WT *base = W + (s_lo + rsub) * p.n + col;
    auto fma_row = [&](const i32x4 &wv, int r) {
        float xv[MAXB];
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) xv[bi] = xs[r * MAXB + bi];
        if constexpr (INT8) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float q = (float)(int8_t)(wv[e >> 2] >> (8 * (e & 3)));
#pragma unroll
                for (int bi = 0; bi < MAXB; ++bi) acc[bi][e] += xv[bi] * q;
            }
        } else {
            const f32x4 wf = __builtin_bit_cast(f32x4, wv);
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[bi][e] += xv[bi] * wf[e];
        }
    };
    int r0 = wb;
    // The first batch of weights does not depend on x: request it before
    // staging x, so the staging latency hides under the weight loads.
    const bool first_full = full_cols && wb + 4 * U <= we;
    i32x4 w0[U];
    if (first_full) {
#pragma unroll
        for (int u = 0; u < U; ++u) w0[u] = *reinterpret_cast<const i32x4 *>(base + (int64_t)(wb + 4 * u) * p.n);
    }
    // Stage this slice's x (times the row scale for int8); for int8 with
    // zero points also sum xs * zp over the slice per batch row -- the
    // column-independent zero-point term.
    float zpart[MAXB];
#pragma unroll
    for (int bi = 0; bi < MAXB; ++bi) zpart[bi] = 0.f;
    for (int r = threadIdx.x; r < rows; r += kThreads) {
        const float sr = INT8 ? p.scales[s_lo + r] : 1.f;
        const float zr = (INT8 && p.zps) ? (float)p.zps[s_lo + r] : 0.f;
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) {
            const float v = bi < nb ? (INT8 ? p.x[bi * p.k + s_lo + r] * sr : p.x[bi * p.k + s_lo + r]) : 0.f;
            xs[r * MAXB + bi] = v;
            zpart[bi] += v * zr;
        }
    }
    if (INT8) {
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) {
            float v = zpart[bi];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0) zred[wave][bi] = v;
        }
    }
    __syncthreads();
    if (first_full) {
#pragma unroll
        for (int u = 0; u < U; ++u) fma_row(w0[u], wb + 4 * u + rsub);
        r0 += 4 * U;
        // Whole batches: no per-row checks.
        for (; r0 + 4 * U <= we; r0 += 4 * U) {
            i32x4 w[U];
#pragma unroll
            for (int u = 0; u < U; ++u) w[u] = *reinterpret_cast<const i32x4 *>(base + (int64_t)(r0 + 4 * u) * p.n);
#pragma unroll
            for (int u = 0; u < U; ++u) fma_row(w[u], r0 + 4 * u + rsub);
        }
    }
    // Remaining rows, ragged columns or unaligned rows: checked loads.
    for (; r0 < we; r0 += 4 * U) {
        i32x4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = r0 + 4 * u;  // this lane's row is r + rsub
            i32x4 v = {0, 0, 0, 0};
            if (r + rsub < we) {
                const WT *src = base + (int64_t)r * p.n;
                if (full_cols) {
                    v = *reinterpret_cast<const i32x4 *>(src);
                } else {
                    WT tmp[EPL];
#pragma unroll
                    for (int e = 0; e < EPL; ++e) tmp[e] = (col + e < p.n) ? src[e] : WT(0);
                    __builtin_memcpy(&v, tmp, 16);
                }
            }
            w[u] = v;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (r0 + 4 * u + rsub < we) fma_row(w[u], r0 + 4 * u + rsub);
    }

    // Reduce over the 4 row lanes of each column group, then over waves.
#pragma unroll
    for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float v = acc[bi][e];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[bi][e] = v;
        }
    if (lane < 16) {
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
            for (int e = 0; e < EPL; ++e) red[wave][bi][lane * EPL + e] = acc[bi][e];
    }
    __syncthreads();
    auto strip_value = [&](int bi, int c) {
        float v = red[0][bi][c];
#pragma unroll
        for (int w2 = 1; w2 < kWaves; ++w2) v = v + red[w2][bi][c];
        if (INT8) v = v - ((zred[0][bi] + zred[1][bi]) + (zred[2][bi] + zred[3][bi]));
        return v;
    };

    if (p.slices == 1) {
        for (int t = threadIdx.x; t < MAXB * SCOLS; t += kThreads) {
            const int bi = t / SCOLS, c = t % SCOLS;
            if (bi >= nb || col0 + c >= p.n) continue;
            p.y[bi * p.n + col0 + c] = strip_value(bi, c);
        }
        return;
    }

    // Split K: publish this slice's partial strip, count arrivals; the last
    // workgroup of the strip sums the slices in order.  Every access to data
    // shared between workgroups (partials, counter) is an agent-scope atomic:
    // such loads and stores go to the device coherence point instead of an
    // XCD's L2, so no L2 writeback or invalidate is needed -- only that the
    // partial stores have completed (vmcnt 0) before the arrival is counted.
    for (int t = threadIdx.x; t < MAXB * SCOLS; t += kThreads) {
        const int bi = t / SCOLS, c = t % SCOLS;
        if (bi >= nb || col0 + c >= p.n) continue;
        __hip_atomic_store(p.part + (slice * nb + bi) * p.n + col0 + c, strip_value(bi, c), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(p.counters + strip, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = (old == (int)p.slices - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // All slice partials are requested before the first is added, in
    // groups of kSumGroup, so the loads overlap instead of paying one memory
    // latency per slice; the sum itself runs in slice order.
    constexpr int kSumGroup = 16;
    for (int t = threadIdx.x; t < MAXB * SCOLS; t += kThreads) {
        const int bi = t / SCOLS, c = t % SCOLS;
        if (bi >= nb || col0 + c >= p.n) continue;
        const float *src = p.part + bi * p.n + col0 + c;
        float v = 0.f;
        for (int64_t j0 = 0; j0 < p.slices; j0 += kSumGroup) {
            float pv[kSumGroup];
#pragma unroll
            for (int j = 0; j < kSumGroup; ++j)
                pv[j] = (j0 + j < p.slices)
                            ? __hip_atomic_load(src + (j0 + j) * nb * p.n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : 0.f;
#pragma unroll
            for (int j = 0; j < kSumGroup; ++j)
                if (j0 + j < p.slices) v = (j0 + j == 0) ? pv[j] : v + pv[j];
        }
        p.y[bi * p.n + col0 + c] = v;
    }
    if (threadIdx.x == 0) __hip_atomic_store(p.counters + strip, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename WT, int MAXB>
void launch_one(const GemvParams &p, bool vec, hipStream_t s) {
    // int8 at b >= 4 is VALU-heavy (b FMAs per weight): fewer rows per
    // batch keep registers low enough for two waves per SIMD.
    constexpr int U = (sizeof(WT) == 1 && MAXB >= 4) ? 4 : 8;
    const dim3 grid((unsigned)(p.nstrips * p.slices)), block(kThreads);
    if (vec)
        hipLaunchKernelGGL((gemv_kernel<WT, MAXB, U, true>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((gemv_kernel<WT, MAXB, U, false>), grid, block, 0, s, p);
}

// Rows per K-slice: 512 (measured best at the BASELINE shapes for both
// weight types: each wave then runs 4 whole batches of 32 rows), halved
// while there would be fewer than ~448 workgroups (each CU streams only
// ~30-45 GB/s, so all CUs must take part), at least 128 rows, a multiple of
// 128 -- and enlarged so the partial strips written and read back stay
// under ~10% of the weight bytes (5% for groups of 8 batch rows, whose
// VALU-heavy slices gain more from fewer, longer slices), up to kMaxSlice.
int64_t choose_kslice(int64_t nstrips, int64_t k, int64_t b, size_t wsize) {
    int64_t ks = 512;
    while (ks > 128 && nstrips * ((k + ks - 1) / ks) < 448) ks /= 2;
    const int64_t nb = b < 8 ? b : 8;
    const double cap = nb >= 8 ? 0.05 : 0.10;
    const int64_t max_slices = (int64_t)(cap * (double)k * (double)wsize / (8.0 * (double)nb));
    if (max_slices >= 1) ks = std::max(ks, (k + max_slices - 1) / max_slices);
    else ks = k;
    ks = (ks + 127) & ~(int64_t)127;
    return std::min<int64_t>(ks, kMaxSlice);
}

template <typename WT>
int launch_gemv(const float *x, const void *w, const float *scales, const int8_t *zps, float *y, int64_t b,
                int64_t k, int64_t n, hipStream_t s) {
    constexpr int SCOLS = kStripBytes / sizeof(WT);
    GemvParams p{};
    p.x = x;
    p.w = w;
    p.scales = scales;
    p.zps = zps;
    p.k = k;
    p.n = n;
    p.nstrips = (n + SCOLS - 1) / SCOLS;
    p.kslice = k > 0 ? choose_kslice(p.nstrips, k, b, sizeof(WT)) : 16;
    p.slices = k > 0 ? (k + p.kslice - 1) / p.kslice : 1;
    if (p.slices > 1) {
        const int64_t gb = b < 8 ? b : 8;
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(float) * (size_t)(p.slices * gb * n), &ws));
        p.part = static_cast<float *>(ws);
        GFH_TRY(stream_counters(s, (size_t)p.nstrips, &p.counters));
    }
    const bool vec = (n * sizeof(WT)) % 16 == 0 && aligned16(w);
    // The batch is processed in groups of at most 8 rows; groups run one
    // after another on the stream, so they share the workspace.
    for (int64_t b0 = 0; b0 < b; b0 += 8) {
        GemvParams q = p;
        const int64_t nbg = (b - b0) < 8 ? (b - b0) : 8;
        q.x = x + b0 * k;
        q.y = y + b0 * n;
        q.b = nbg;
        if (nbg == 1)
            launch_one<WT, 1>(q, vec, s);
        else if (nbg == 2)
            launch_one<WT, 2>(q, vec, s);
        else if (nbg <= 4)
            launch_one<WT, 4>(q, vec, s);
        else
            launch_one<WT, 8>(q, vec, s);
        GFH_TRY(check_launch(sizeof(WT) == 1 ? "gemv_w8" : "gemv_f32"));
    }
    return GFH_SUCCESS;
}

}  // namespace

int launch_gemv_f32(const float *x, const float *w, float *y, int64_t b, int64_t k, int64_t n, hipStream_t s) {
    return launch_gemv<float>(x, w, nullptr, nullptr, y, b, k, n, s);
}

int launch_gemv_w8(const float *x, const int8_t *qw, const float *scales, const int8_t *zps, float *y, int64_t b,
                   int64_t k, int64_t n, hipStream_t s) {
    return launch_gemv<int8_t>(x, qw, scales, zps, y, b, k, n, s);
}

}  // namespace gfh
