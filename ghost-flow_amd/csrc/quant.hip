// quant.hip -- int8 quantize / dequantize with the reference's scheme
// (ghostflow-nn/src/quantization.rs:77-204), bit-exact:
//   min/max folds ignore NaN (f32::min / f32::max  ->  fminf / fmaxf);
//   symmetric : scale = max(|min|, |max|) / 127, zp = 0
//   asymmetric: scale = (max - min) / 255, zp = ((-min / scale) - 128).round() as i8
//   q = ((x / scale).round() as i32 + zp).clamp(-128, 127)
// `/` is the correctly rounded IEEE f32 division (hipcc's default), `round`
// is half away from zero, `as` casts saturate with NaN -> 0, and the i32 add
// wraps as in a release build.  All kernels are HBM-bound elementwise or
// reduction passes: 16-byte loads, grid sized to fill the 256 CUs.
#include <cstdlib>

#include "common.hpp"
#include "kernels.hpp"
#include "quant_math.hpp"

// Every multiply and add below is its own f32 rounding, as in the reference
// (rustc never contracts a*b+c into an FMA); the MFMA accumulation itself is
// not affected by this pragma.
#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kBlock = 256;

using qmath::quant4;
using qmath::quant_one;
using qmath::quant_params;
using qmath::sat_f32_to_i32;
using qmath::sat_f32_to_i8;

__device__ __forceinline__ void block_minmax(float &mn, float &mx) { qmath::block_minmax<kBlock>(mn, mx); }

// ---- per channel: one workgroup per row --------------------------------------
template <bool VEC>
__global__ __launch_bounds__(kBlock) void quant_per_channel_kernel(const float *__restrict__ x, int64_t cols,
                                                                  bool symmetric, int8_t *__restrict__ q,
                                                                  float *__restrict__ scales,
                                                                  int8_t *__restrict__ zps) {
    const int64_t row = blockIdx.x;
    const float *xr = x + row * cols;
    int8_t *qr = q + row * cols;
    float mn = INFINITY, mx = -INFINITY;
    if (VEC) {
        const int64_t nv = cols / 4;
        for (int64_t i = threadIdx.x; i < nv; i += kBlock) {
            const f32x4 v = reinterpret_cast<const f32x4 *>(xr)[i];
            mn = fminf(fminf(mn, v[0]), fminf(fminf(v[1], v[2]), v[3]));
            mx = fmaxf(fmaxf(mx, v[0]), fmaxf(fmaxf(v[1], v[2]), v[3]));
        }
    } else {
        for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
            mn = fminf(mn, xr[i]);
            mx = fmaxf(mx, xr[i]);
        }
    }
    block_minmax(mn, mx);
    float scale;
    int8_t zp;
    quant_params(mn, mx, symmetric, scale, zp);
    if (threadIdx.x == 0) {
        scales[row] = scale;
        zps[row] = zp;
    }
    if (VEC) {
        const int64_t nv = cols / 4;
        for (int64_t i = threadIdx.x; i < nv; i += kBlock)
            reinterpret_cast<uint32_t *>(qr)[i] = quant4(reinterpret_cast<const f32x4 *>(xr)[i], scale, zp);
    } else {
        for (int64_t i = threadIdx.x; i < cols; i += kBlock) qr[i] = quant_one(xr[i], scale, zp);
    }
}

// ---- per tensor: partial min/max, then finalize + quantize ---------------------
constexpr int kMaxPartials = 1024;
// float4s per thread per partial block: 4096 elements per workgroup, so
// 256 workgroups cover a [256, 4096] activation (with 8, 128 did, and the
// two passes took 12.6 us for its 4 MB).
constexpr int64_t kVecPerThread = 4;
// float4 loads a thread has in flight per loop step (all issued before the
// first is used).
constexpr int kUnroll = 4;

int per_tensor_blocks(int64_t n) {
    const int64_t per_block = (int64_t)kBlock * 4 * kVecPerThread;
    int64_t nb = (n + per_block - 1) / per_block;
    if (nb < 1) nb = 1;
    if (nb > kMaxPartials) nb = kMaxPartials;
    return (int)nb;
}

template <bool VEC>
__global__ __launch_bounds__(kBlock) void minmax_partial_kernel(const float *__restrict__ x, int64_t n,
                                                               float2 *__restrict__ partials) {
    float mn = INFINITY, mx = -INFINITY;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    if (VEC) {
        const int64_t nv = n / 4;
        const f32x4 *xv = reinterpret_cast<const f32x4 *>(x);
        int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
        for (; i + (kUnroll - 1) * stride < nv; i += kUnroll * stride) {
            f32x4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) v[u] = xv[i + u * stride];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                mn = fminf(fminf(mn, v[u][0]), fminf(fminf(v[u][1], v[u][2]), v[u][3]));
                mx = fmaxf(fmaxf(mx, v[u][0]), fmaxf(fmaxf(v[u][1], v[u][2]), v[u][3]));
            }
        }
        for (; i < nv; i += stride) {
            const f32x4 v = xv[i];
            mn = fminf(fminf(mn, v[0]), fminf(fminf(v[1], v[2]), v[3]));
            mx = fmaxf(fmaxf(mx, v[0]), fmaxf(fmaxf(v[1], v[2]), v[3]));
        }
        for (int64_t i = nv * 4 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
            mn = fminf(mn, x[i]);
            mx = fmaxf(mx, x[i]);
        }
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
            mn = fminf(mn, x[i]);
            mx = fmaxf(mx, x[i]);
        }
    }
    block_minmax(mn, mx);
    if (threadIdx.x == 0) partials[blockIdx.x] = make_float2(mn, mx);
}

template <bool VEC>
__global__ __launch_bounds__(kBlock) void quant_per_tensor_kernel(const float *__restrict__ x, int64_t n,
                                                                 bool symmetric, const float2 *__restrict__ partials,
                                                                 int npartials, int8_t *__restrict__ q,
                                                                 float *__restrict__ scale_out,
                                                                 int8_t *__restrict__ zp_out) {
    // Every workgroup folds all partials (at most 1024 pairs) itself, so the
    // parameters are identical everywhere without a grid-wide barrier.
    float mn = INFINITY, mx = -INFINITY;
    for (int i = threadIdx.x; i < npartials; i += kBlock) {
        const float2 p = partials[i];
        mn = fminf(mn, p.x);
        mx = fmaxf(mx, p.y);
    }
    block_minmax(mn, mx);
    float scale;
    int8_t zp;
    quant_params(mn, mx, symmetric, scale, zp);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *scale_out = scale;
        *zp_out = zp;
    }
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    if (VEC) {
        const int64_t nv = n / 4;
        const f32x4 *xv = reinterpret_cast<const f32x4 *>(x);
        uint32_t *qv = reinterpret_cast<uint32_t *>(q);
        int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
        for (; i + (kUnroll - 1) * stride < nv; i += kUnroll * stride) {
            f32x4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) v[u] = xv[i + u * stride];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) qv[i + u * stride] = quant4(v[u], scale, zp);
        }
        for (; i < nv; i += stride) qv[i] = quant4(xv[i], scale, zp);
        for (int64_t i = nv * 4 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
            q[i] = quant_one(x[i], scale, zp);
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
            q[i] = quant_one(x[i], scale, zp);
    }
}

// ---- small tensors in one launch ---------------------------------------------
// Up to kResMaxGroups workgroups of 1024 threads, each thread holding one
// float4 of x in registers, do both passes in one launch:
//   1. each workgroup loads its share and folds its (min, max);
//   2. it publishes the pair and counts its arrival with the split-K
//      arrival protocol (common.hpp: agent-scope stores, vmcnt(0), agent-scope
//      fetch_add on counters[0]);
//   3. it waits until every workgroup has arrived, then folds all pairs
//      (agent-scope loads), so every workgroup derives the same (scale, zp);
//   4. it writes its codes from the registers.
// counters[1] counts the workgroups done with the pairs; the last one returns
// both counters to 0.  The wait is bounded: it only lasts while a workgroup
// of the grid has not started, which needs other kernels holding every CU.
// A workgroup that gives up waiting folds all of x itself, which gives the
// same (min, max) as the pairs (exact folds; zeros of either sign give the
// same codes), so the codes are right either way and every wave exits.
constexpr int kResThreads = 1024;
constexpr int kResMaxGroups = 16;
// Wait rounds (s_sleep 2, ~128 clocks, plus one agent-scope load of a few
// hundred ns each) before a workgroup gives up: a few ms at most, far above
// the few microseconds the whole grid needs to start when the GPU is free,
// and a bounded cost when other streams hold the CUs (the fold-everything
// path then reads all of x, at most 256 KiB, per workgroup).
// GFH_QUANT_WAIT_ROUNDS lowers it (0: every workgroup takes the
// fold-everything path; used by the tests of that path).
constexpr int kResSpinLimit = 1 << 12;

__global__ __launch_bounds__(kResThreads) void quant_small_kernel(const float *__restrict__ x, int64_t n,
                                                                 bool symmetric, float *__restrict__ partials,
                                                                 int *__restrict__ counters, int8_t *__restrict__ q,
                                                                 float *__restrict__ scale_out,
                                                                 int8_t *__restrict__ zp_out, int spin_limit) {
    const int tid = threadIdx.x;
    const int nwg = gridDim.x;
    const int nfull4 = (int)(n / 4);  // kResThreads <= nfull4 <= kResThreads * kResMaxGroups (host check)
    const int i4 = blockIdx.x * kResThreads + tid;
    const f32x4 *xv = reinterpret_cast<const f32x4 *>(x);
    // Load from a clamped index; past the last whole float4 the elements are
    // replaced afterwards (NaN is neutral for the NaN-ignoring folds).
    f32x4 v = xv[i4 < nfull4 ? i4 : nfull4 - 1];
    if (i4 >= nfull4) {
        float e[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) e[c] = (int64_t)i4 * 4 + c < n ? x[(int64_t)i4 * 4 + c] : NAN;
        v = f32x4{e[0], e[1], e[2], e[3]};
    }
    float mn = fminf(fminf(v[0], v[1]), fminf(v[2], v[3]));
    float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    qmath::block_minmax<kResThreads>(mn, mx);

    __shared__ int s_gave_up;
    if (tid == 0) {
        __hip_atomic_store(partials + 2 * blockIdx.x, mn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(partials + 2 * blockIdx.x + 1, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the pair is at the coherence point
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // Its return value is waited for: this arrival is counted before the
        // wait, and before counters[1] below.
        int arrived = __hip_atomic_fetch_add(counters, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
        for (int spin = 0; arrived < nwg && spin < spin_limit; ++spin) {
            __builtin_amdgcn_s_sleep(2);
            arrived = __hip_atomic_load(counters, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_gave_up = arrived < nwg;
    }
    __syncthreads();
    float gmn = INFINITY, gmx = -INFINITY;
    if (!s_gave_up) {
        if (tid < nwg) {
            gmn = __hip_atomic_load(partials + 2 * tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            gmx = __hip_atomic_load(partials + 2 * tid + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        for (int64_t i = tid; i < n; i += kResThreads) {
            gmn = fminf(gmn, x[i]);
            gmx = fmaxf(gmx, x[i]);
        }
    }
    qmath::block_minmax<kResThreads>(gmn, gmx);  // its barrier: every load above has been used
    if (tid == 0) {
        const int done = __hip_atomic_fetch_add(counters + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == nwg - 1) {  // every workgroup has left the wait
            __hip_atomic_store(counters, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(counters + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    float scale;
    int8_t zp;
    quant_params(gmn, gmx, symmetric, scale, zp);
    if (blockIdx.x == 0 && tid == 0) {
        *scale_out = scale;
        *zp_out = zp;
    }
    if (i4 < nfull4) {
        reinterpret_cast<uint32_t *>(q)[i4] = quant4(v, scale, zp);
    } else {
        const float e[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if ((int64_t)i4 * 4 + c < n) q[(int64_t)i4 * 4 + c] = quant_one(e[c], scale, zp);
    }
}

// Workgroups of the one-launch form for n elements, or 0 when n is outside
// its range.  Measured (µs, one launch / two): 16384 elements 5.7 / 6.5-7.0;
// at 262144 (64 workgroups) 7.9 / 7.0, and larger grids lose more.
int small_groups(int64_t n) {
    if (n < 4 * (int64_t)kResThreads) return 0;
    const int64_t g = ((n + 3) / 4 + kResThreads - 1) / kResThreads;
    return g <= kResMaxGroups ? (int)g : 0;
}

int spin_limit() {
    const char *e = getenv("GFH_QUANT_WAIT_ROUNDS");
    if (e == nullptr || *e == '\0') return kResSpinLimit;
    const long v = strtol(e, nullptr, 10);
    return v < 0 ? 0 : (v > kResSpinLimit ? kResSpinLimit : (int)v);
}

// ---- dequantize -------------------------------------------------------------------
// out = ((float)q - (float)zp) * scale, per tensor (nscales == 1) or per row.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void dequant_kernel(const int8_t *__restrict__ q, int64_t rows, int64_t cols,
                                                        const float *__restrict__ scales,
                                                        const int8_t *__restrict__ zps, bool per_row,
                                                        float *__restrict__ out) {
    const int64_t n = rows * cols;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    if (VEC) {  // cols % 4 == 0: a group of 4 never straddles two rows
        const int64_t nv = n / 4;
        for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < nv; i += stride) {
            const int64_t g = per_row ? (i * 4) / cols : 0;
            const float s = scales[g];
            const float z = (float)zps[g];
            const uint32_t packed = reinterpret_cast<const uint32_t *>(q)[i];
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = ((float)(int8_t)(packed >> (8 * e)) - z) * s;
            reinterpret_cast<f32x4 *>(out)[i] = v;
        }
    } else {
        for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
            const int64_t g = per_row ? i / cols : 0;
            out[i] = ((float)q[i] - (float)zps[g]) * scales[g];
        }
    }
}

// ---- int8 row sums ------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void rowsum_i8_kernel(const int8_t *__restrict__ q, int64_t n, int64_t k,
                                                          int32_t *__restrict__ out) {
    // one wave per row
    const int64_t row = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const int8_t *r = q + row * k;
    int32_t s = 0;
    for (int64_t i = lane; i < k; i += 64) s += r[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) out[row] = s;
}

int grid_for(int64_t work_items) {
    int64_t g = (work_items + kBlock - 1) / kBlock;
    if (g < 1) g = 1;
    if (g > 8192) g = 8192;
    return (int)g;
}

}  // namespace

int launch_quantize_per_channel(const float *x, int64_t rows, int64_t cols, bool symmetric, int8_t *q,
                                float *scales, int8_t *zps, hipStream_t s) {
    const bool vec = (cols % 4 == 0) && aligned16(x) && ((reinterpret_cast<uintptr_t>(q) & 3u) == 0);
    if (vec)
        hipLaunchKernelGGL(quant_per_channel_kernel<true>, dim3((unsigned)rows), dim3(kBlock), 0, s, x, cols,
                           symmetric, q, scales, zps);
    else
        hipLaunchKernelGGL(quant_per_channel_kernel<false>, dim3((unsigned)rows), dim3(kBlock), 0, s, x, cols,
                           symmetric, q, scales, zps);
    return check_launch("quantize_per_channel");
}

size_t quantize_per_tensor_workspace(int64_t n) { return sizeof(float2) * (size_t)per_tensor_blocks(n); }

int launch_quantize_per_tensor(const float *x, int64_t n, bool symmetric, int8_t *q, float *scale, int8_t *zp,
                               void *ws, hipStream_t s) {
    const int nb = per_tensor_blocks(n);
    float2 *partials = static_cast<float2 *>(ws);
    const bool vec = aligned16(x) && ((reinterpret_cast<uintptr_t>(q) & 3u) == 0);
    const int groups = vec ? small_groups(n) : 0;
    if (groups) {
        // One launch; its grid never exceeds nb, so the workspace holds its pairs.
        int *counters = nullptr;
        GFH_TRY(stream_counters(s, 2, &counters));
        hipLaunchKernelGGL(quant_small_kernel, dim3(groups), dim3(kResThreads), 0, s, x, n, symmetric,
                           reinterpret_cast<float *>(partials), counters, q, scale, zp, spin_limit());
        return check_launch("quantize_per_tensor/one_launch");
    }
    if (vec) {
        hipLaunchKernelGGL(minmax_partial_kernel<true>, dim3(nb), dim3(kBlock), 0, s, x, n, partials);
        GFH_TRY(check_launch("quantize_per_tensor/minmax"));
        hipLaunchKernelGGL(quant_per_tensor_kernel<true>, dim3(nb), dim3(kBlock), 0, s, x, n, symmetric, partials,
                           nb, q, scale, zp);
    } else {
        hipLaunchKernelGGL(minmax_partial_kernel<false>, dim3(nb), dim3(kBlock), 0, s, x, n, partials);
        GFH_TRY(check_launch("quantize_per_tensor/minmax"));
        hipLaunchKernelGGL(quant_per_tensor_kernel<false>, dim3(nb), dim3(kBlock), 0, s, x, n, symmetric,
                           partials, nb, q, scale, zp);
    }
    return check_launch("quantize_per_tensor/quantize");
}

// The quantize pass alone, on (min, max) partials a producer kernel already
// wrote (the fused SwiGLU gate/up kernel does, one per workgroup).
int launch_quantize_per_tensor_partials(const float *x, int64_t n, bool symmetric, const float2 *partials,
                                       int npartials, int8_t *q, float *scale, int8_t *zp, hipStream_t s) {
    const int nb = per_tensor_blocks(n);
    const bool vec = aligned16(x) && ((reinterpret_cast<uintptr_t>(q) & 3u) == 0);
    if (vec)
        hipLaunchKernelGGL(quant_per_tensor_kernel<true>, dim3(nb), dim3(kBlock), 0, s, x, n, symmetric, partials,
                           npartials, q, scale, zp);
    else
        hipLaunchKernelGGL(quant_per_tensor_kernel<false>, dim3(nb), dim3(kBlock), 0, s, x, n, symmetric, partials,
                           npartials, q, scale, zp);
    return check_launch("quantize_per_tensor/quantize");
}

int launch_dequantize(const int8_t *q, int64_t rows, int64_t cols, const float *scales, const int8_t *zps,
                      int64_t nscales, float *out, hipStream_t s) {
    const bool per_row = nscales != 1;
    const bool vec = (cols % 4 == 0) && aligned16(out) && ((reinterpret_cast<uintptr_t>(q) & 3u) == 0);
    const int64_t n = rows * cols;
    if (vec)
        hipLaunchKernelGGL(dequant_kernel<true>, dim3(grid_for(n / 4)), dim3(kBlock), 0, s, q, rows, cols, scales,
                           zps, per_row, out);
    else
        hipLaunchKernelGGL(dequant_kernel<false>, dim3(grid_for(n)), dim3(kBlock), 0, s, q, rows, cols, scales,
                           zps, per_row, out);
    return check_launch("dequantize");
}

int launch_rowsum_i8(const int8_t *q, int64_t n, int64_t k, int32_t *rowsum, hipStream_t s) {
    const int64_t blocks = (n + (kBlock / 64) - 1) / (kBlock / 64);
    hipLaunchKernelGGL(rowsum_i8_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s, q, n, k, rowsum);
    return check_launch("qweight_rowsum");
}

}  // namespace gfh
