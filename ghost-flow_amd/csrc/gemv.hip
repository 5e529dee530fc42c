// gemv.hip -- batched decode GEMV, HBM-bound: y[b,n] = sum_k x[b,k] * W[k,n]
// for W [K, N] row-major (Tensor::matmul with M = b,
// ghostflow-core/src/ops/matmul.rs:91-119), fp32 or int8 weights.
//
// The int8 form is DynamicQuantization::get_weights -> Tensor::matmul
// (ghostflow-nn/src/quantization.rs:173-204, :275-277) fused: every weight
// is dequantized in registers to exactly the reference's value
// fl((q - zp[k]) * s[k]) and never written to memory.
//
// Layout of the work:
//  * A wave reads one row of W at a time across 256 contiguous columns
//    (lane l owns columns c0 + 4l .. +3: a 16-byte load for f32, 4 bytes for
//    int8), so each wave-wide load is one contiguous 1 KB / 256 B run.
//  * Because a whole wave works on the same row k, x[b,k] is wave-uniform
//    and is fetched with scalar loads (the row index is made uniform with
//    readfirstlane), keeping x out of the vector memory path.
//  * Workgroup = 4 waves on one 256-column strip and one K-slice; the waves
//    split the slice, unroll U rows to keep U loads in flight per lane, and
//    combine through LDS in a fixed order.
//  * Grid = strips x S K-slices.  With S > 1 each workgroup writes its
//    partial to a workspace and a second pass adds the S partials in slice
//    order, so results are deterministic run to run.
#include "common.hpp"
#include "kernels.hpp"

namespace gfh {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kCols = 256;  // columns per workgroup strip

struct GemvParams {
    const float *x;
    const void *w;
    const float *scales;
    const int8_t *zps;
    float *out;  // y (S == 1) or partials [S][b][n]
    int64_t b, k, n;
    int64_t kslice;  // rows per K-slice
};

template <int MAXB>
__device__ __forceinline__ void reduce_and_store(float (&acc)[MAXB][4], const GemvParams &p, int64_t col,
                                                 bool full_vec) {
    __shared__ float red[kWaves][MAXB][kCols];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[wave][bi][lane * 4 + e] = acc[bi][e];
    __syncthreads();
    // 256 threads: thread t finishes column t of the strip for every b.
    const int t = threadIdx.x;
    const int64_t c = (col - (int64_t)(lane * 4)) + t;  // strip base + t
    float *dst = p.out + (int64_t)blockIdx.y * p.b * p.n;
    if (c < p.n) {
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) {
            if (bi >= p.b) break;
            float s = red[0][bi][t];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) s = s + red[w][bi][t];
            dst[bi * p.n + c] = s;
        }
    }
    (void)full_vec;
}

// ---- fp32 weights ------------------------------------------------------------
template <int MAXB, int U, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_f32_kernel(GemvParams p) {
    const float *__restrict__ W = static_cast<const float *>(p.w);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t col = (int64_t)blockIdx.x * kCols + lane * 4;
    const int64_t k_lo = (int64_t)blockIdx.y * p.kslice;
    const int64_t k_hi = min(k_lo + p.kslice, p.k);
    const int64_t per_wave = (p.kslice + kWaves - 1) / kWaves;
    const int64_t kb = k_lo + wave * per_wave;
    const int64_t ke = min(kb + per_wave, k_hi);
    const bool full = VEC && (col + 3 < p.n);

    float acc[MAXB][4];
#pragma unroll
    for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[bi][e] = 0.f;

    for (int64_t k0 = kb; k0 < ke; k0 += U) {
        f32x4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t k = k0 + u;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (k < ke) {
                const float *row = W + k * p.n + col;
                if (full) {
                    v = *reinterpret_cast<const f32x4 *>(row);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < p.n) v[e] = row[e];
                }
            }
            w[u] = v;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t k = k0 + u;
            if (k >= ke) break;
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi) {
                if (bi >= p.b) break;
                const float xv = p.x[bi * p.k + k];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[bi][e] = acc[bi][e] + xv * w[u][e];
            }
        }
    }
    reduce_and_store<MAXB>(acc, p, col, full);
}

// ---- int8 weights, per-row (per-k) scale and zero point -----------------------
template <int MAXB, int U, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_w8_kernel(GemvParams p) {
    const int8_t *__restrict__ W = static_cast<const int8_t *>(p.w);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t col = (int64_t)blockIdx.x * kCols + lane * 4;
    const int64_t k_lo = (int64_t)blockIdx.y * p.kslice;
    const int64_t k_hi = min(k_lo + p.kslice, p.k);
    const int64_t per_wave = (p.kslice + kWaves - 1) / kWaves;
    const int64_t kb = k_lo + wave * per_wave;
    const int64_t ke = min(kb + per_wave, k_hi);
    const bool full = VEC && (col + 3 < p.n);

    float acc[MAXB][4];
#pragma unroll
    for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[bi][e] = 0.f;

    for (int64_t k0 = kb; k0 < ke; k0 += U) {
        uint32_t w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t k = k0 + u;
            uint32_t v = 0u;
            if (k < ke) {
                const int8_t *row = W + k * p.n + col;
                if (full) {
                    v = *reinterpret_cast<const uint32_t *>(row);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < p.n) v |= (uint32_t)(uint8_t)row[e] << (8 * e);
                }
            }
            w[u] = v;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t k = k0 + u;
            if (k >= ke) break;
            const float s = p.scales[k];
            const float z = p.zps ? (float)p.zps[k] : 0.f;
            // dequantize_int8: (q as f32 - zp as f32) * scale, exact reference value
            float wv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) wv[e] = ((float)(int8_t)(w[u] >> (8 * e)) - z) * s;
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi) {
                if (bi >= p.b) break;
                const float xv = p.x[bi * p.k + k];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[bi][e] = acc[bi][e] + xv * wv[e];
            }
        }
    }
    reduce_and_store<MAXB>(acc, p, col, full);
}

// y[b, n] = sum over s of partials[s][b][n], slices in order.
__global__ __launch_bounds__(kThreads) void sum_partials_kernel(const float *__restrict__ part, int64_t slices,
                                                               int64_t count, float *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= count) return;
    float s = part[i];
    for (int64_t j = 1; j < slices; ++j) s = s + part[j * count + i];
    y[i] = s;
}

// Number of K-slices: enough workgroups to cover the 256 CUs about twice,
// each slice at least 256 rows.
int64_t choose_slices(int64_t k, int64_t n) {
    const int64_t strips = (n + kCols - 1) / kCols;
    int64_t s = 1;
    while (strips * s < 512 && k / (s * 2) >= 256) s *= 2;
    return s;
}

template <bool INT8, int MAXB>
void launch_one(const GemvParams &p, dim3 grid, bool vec, hipStream_t s) {
    constexpr int U = INT8 ? 16 : 8;
    if constexpr (INT8) {
        if (vec)
            hipLaunchKernelGGL((gemv_w8_kernel<MAXB, U, true>), grid, dim3(kThreads), 0, s, p);
        else
            hipLaunchKernelGGL((gemv_w8_kernel<MAXB, U, false>), grid, dim3(kThreads), 0, s, p);
    } else {
        if (vec)
            hipLaunchKernelGGL((gemv_f32_kernel<MAXB, U, true>), grid, dim3(kThreads), 0, s, p);
        else
            hipLaunchKernelGGL((gemv_f32_kernel<MAXB, U, false>), grid, dim3(kThreads), 0, s, p);
    }
}

template <bool INT8>
int launch_gemv(const float *x, const void *w, const float *scales, const int8_t *zps, float *y, int64_t b,
                int64_t k, int64_t n, hipStream_t s) {
    const int64_t strips = (n + kCols - 1) / kCols;
    const int64_t slices = k > 0 ? choose_slices(k, n) : 1;
    Scratch ws;
    float *out = y;
    if (slices > 1) {
        GFH_TRY(ws.acquire(nullptr, 0, sizeof(float) * (size_t)(slices * b * n), s));
        out = static_cast<float *>(ws.ptr());
    }
    GemvParams p{};
    p.x = x;
    p.w = w;
    p.scales = scales;
    p.zps = zps;
    p.out = out;
    p.b = b;
    p.k = k;
    p.n = n;
    p.kslice = k > 0 ? (k + slices - 1) / slices : 1;
    const bool vec = (n % 4 == 0) && (INT8 ? (reinterpret_cast<uintptr_t>(w) & 3u) == 0 : aligned16(w));
    dim3 grid((unsigned)strips, (unsigned)slices);
    // Process the batch in groups of at most 8 rows (registers hold 8 x 4 sums).
    for (int64_t b0 = 0; b0 < b; b0 += 8) {
        GemvParams q = p;
        const int64_t nb = (b - b0) < 8 ? (b - b0) : 8;
        q.x = x + b0 * k;
        q.b = nb;
        // partial layout for this group: [slices][nb][n] inside the workspace
        q.out = slices > 1 ? out + b0 * n * slices : y + b0 * n;
        if (nb == 1)
            launch_one<INT8, 1>(q, grid, vec, s);
        else if (nb == 2)
            launch_one<INT8, 2>(q, grid, vec, s);
        else if (nb <= 4)
            launch_one<INT8, 4>(q, grid, vec, s);
        else
            launch_one<INT8, 8>(q, grid, vec, s);
        GFH_TRY(check_launch(INT8 ? "gemv_w8" : "gemv_f32"));
        if (slices > 1) {
            const int64_t count = nb * n;
            hipLaunchKernelGGL(sum_partials_kernel, dim3((unsigned)((count + kThreads - 1) / kThreads)),
                               dim3(kThreads), 0, s, (const float *)q.out, slices, count, y + b0 * n);
            GFH_TRY(check_launch("gemv/sum_partials"));
        }
    }
    return GFH_SUCCESS;
}

}  // namespace

int launch_gemv_f32(const float *x, const float *w, float *y, int64_t b, int64_t k, int64_t n, hipStream_t s) {
    return launch_gemv<false>(x, w, nullptr, nullptr, y, b, k, n, s);
}

int launch_gemv_w8(const float *x, const int8_t *qw, const float *scales, const int8_t *zps, float *y, int64_t b,
                   int64_t k, int64_t n, hipStream_t s) {
    return launch_gemv<true>(x, qw, scales, zps, y, b, k, n, s);
}

}  // namespace gfh
