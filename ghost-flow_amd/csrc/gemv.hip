// gemv.hip -- batched decode GEMV, HBM-bound: y[b,n] = sum_k x[b,k] * W[k,n]
// for W [K, N] row-major (Tensor::matmul with M = b,
// ghostflow-core/src/ops/matmul.rs:91-119), fp32 or int8 weights.
//
// The int8 form is DynamicQuantization::get_weights -> Tensor::matmul
// (ghostflow-nn/src/quantization.rs:173-204, :275-277) without ever
// materializing the fp32 weight:
//   y[b,n] = sum_k x[b,k] * ((q[k,n] - zp[k]) * s[k]) = sum_k xs[b,k] * (q[k,n] - zp[k]),
// xs = x * s[k].  (The products are regrouped, so the result is within the
// fp32 GEMM bound of the reference, not bit-identical to it.)
//
// Layout of the work (one kernel per group of up to 8 batch rows):
//  * A workgroup (4 wave64) owns a strip of 256 bytes of every W row (64
//    fp32 or 256 int8 columns) over one K-slice; every load instruction
//    covers 4 rows x 256 contiguous bytes (HBM streams 256-byte row runs at
//    about 6 TB/s; 128-byte runs only reach ~5).  The slice's activations
//    are staged in LDS once per workgroup (fp32 with aligned x: streamed
//    with the weights instead, a step's rows at a time).
//  * fp32 (gemv_f32_kernel): lane l reads 16 bytes of row l/16 of a 4-row
//    group and the b multiply-adds run on the VALU; partial sums are reduced
//    over the 4 row lanes with xor shuffles, then over the waves in LDS.
//    With at most one workgroup per CU it runs 8 waves, twice the bytes in
//    flight per CU (W [4096, 14336], 1 batch row: 41.5 against 42.9 us).
//  * int8 (w8mf::gemv_w8_mfma_kernel): the weights become exact f16 and the
//    multiply-adds run on the matrix cores (v_mfma_f32_16x16x32_f16), so
//    batches of 1-8 rows cost the same.
//  * K is split into S slices when the strips alone are too few workgroups:
//    every workgroup writes its partial strip to a workspace, and the last
//    of the S to finish (an agent-scope arrival counter) adds the S
//    partials in slice order and writes y -- deterministic, one launch.  The
//    counter is returned to 0 by that last workgroup.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

// No implicit contraction of a*b+c: where this file writes a separate
// product and sum they round separately.  The fp32 accumulation itself is
// deliberately fused -- explicit fmaf on the VALU path and MFMA on the
// matrix-core paths -- under the GEMM error bound the tests apply, not
// the reference's separate roundings.
#pragma clang fp contract(off)

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
    int xvec;        // x rows 16-byte aligned and k % 4 == 0 (fp32 kernel: staged 4 rows per load)
    int off32;       // the weight is under 4 GB: byte offsets into it fit 32 bits
    // gfh_sgemm's epilogue when it routes a product here (epi != 0):
    // y = alpha * (x . W), then + beta * y, then + bias, each rounded
    float alpha, beta;
    const float *bias;
    int epi;
};

// The value stored for batch row bi, column col of y, from the product v.
__device__ __forceinline__ float gemv_out(const GemvParams &p, int64_t bi, int64_t col, float v) {
    if (!p.epi) return v;
    float o = p.alpha * v;
    if (p.beta != 0.f) o = o + p.beta * p.y[bi * p.n + col];
    if (p.bias) o = o + p.bias[col];
    return o;
}

constexpr int kMaxSlice = 1024;  // int8 kernel

// Rows per slice the fp32 kernel can stage: its activations take
// rows x MAXB floats of LDS (static, so it also bounds the workgroups per
// CU).  4096 rows (16 per thread) up to 4 batch rows -- one slice for
// K = 4096 -- and 1024 for 8 batch rows, whose slices are split anyway:
// 2048 rows there (64 KB) measured 55.1 us against 50.8 at 1024 (32 KB).
template <int MAXB>
constexpr int f32_max_rows() { return MAXB >= 8 ? 1024 : 4096; }

// Writes this workgroup's strip -- value(bi, c) for batch row bi < nb and
// strip column c -- to y when K is not split.  Otherwise publishes it as the
// slice's partial strip and counts arrivals; the last workgroup of the strip
// to arrive sums the slices in order.  Every access to data shared between
// workgroups (partials, counter) is an agent-scope atomic: such loads and
// stores go to the device coherence point instead of an XCD's L2, so no L2
// writeback or invalidate is needed -- only that the partial stores have
// completed (vmcnt 0) before the arrival is counted.  The counter is
// returned to 0 by that last workgroup.
// EPI: the fp32 kernel, whose callers may ask for gfh_sgemm's epilogue (the
// int8 kernel never stores through it, and its 8-row form measured 8% slower
// with the check compiled in).
template <int MAXB, int SCOLS, int NT = kThreads, bool EPI = false, typename F>
__device__ __forceinline__ void store_strip(const GemvParams &p, int64_t strip, int64_t slice, int64_t nb,
                                            int64_t col0, int *last_flag, F value) {
    if (p.slices == 1) {
        for (int t = threadIdx.x; t < MAXB * SCOLS; t += NT) {
            const int bi = t / SCOLS, c = t % SCOLS;
            if (bi >= nb || col0 + c >= p.n) continue;
            p.y[bi * p.n + col0 + c] = EPI ? gemv_out(p, bi, col0 + c, value(bi, c)) : value(bi, c);
        }
        return;
    }

    for (int t = threadIdx.x; t < MAXB * SCOLS; t += NT) {
        const int bi = t / SCOLS, c = t % SCOLS;
        if (bi >= nb || col0 + c >= p.n) continue;
        __hip_atomic_store(p.part + (slice * nb + bi) * p.n + col0 + c, value(bi, c), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    // split-K arrival protocol (common.hpp): steps 2-4
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(p.counters + strip, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last_flag = (old == (int)p.slices - 1);
    }
    __syncthreads();
    if (!*last_flag) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // Each thread requests the partials of all its outputs, for a group of
    // slices at a time, before adding any of them, so the loads overlap
    // instead of paying one memory latency per output or slice; each output
    // is still summed in slice order.
    constexpr int kOut = (MAXB * SCOLS + NT - 1) / NT;  // outputs per thread
    constexpr int kGroup = kOut >= 32 ? 1 : 32 / kOut;                // slices per group
    const float *src[kOut];
    float v[kOut];
#pragma unroll
    for (int o = 0; o < kOut; ++o) {
        const int t = threadIdx.x + o * NT;
        const int bi = t / SCOLS, c = t % SCOLS;
        const bool ok = t < MAXB * SCOLS && bi < nb && col0 + c < p.n;
        src[o] = ok ? p.part + bi * p.n + col0 + c : nullptr;
        v[o] = 0.f;
    }
    for (int64_t j0 = 0; j0 < p.slices; j0 += kGroup) {
        float pv[kOut][kGroup];
#pragma unroll
        for (int o = 0; o < kOut; ++o)
#pragma unroll
            for (int j = 0; j < kGroup; ++j)
                pv[o][j] = (src[o] && j0 + j < p.slices)
                               ? __hip_atomic_load(src[o] + (j0 + j) * nb * p.n, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                               : 0.f;
#pragma unroll
        for (int o = 0; o < kOut; ++o)
#pragma unroll
            for (int j = 0; j < kGroup; ++j)
                if (j0 + j < p.slices) v[o] = (j0 + j == 0) ? pv[o][j] : v[o] + pv[o][j];
    }
#pragma unroll
    for (int o = 0; o < kOut; ++o)
        if (src[o]) {
            const int t = threadIdx.x + o * NT;
            p.y[(t / SCOLS) * p.n + col0 + t % SCOLS] = EPI ? gemv_out(p, t / SCOLS, col0 + t % SCOLS, v[o]) : v[o];
        }
    if (threadIdx.x == 0) __hip_atomic_store(p.counters + strip, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// NW waves per workgroup: 8 when the grid has at most one workgroup per CU,
// so that twice the weight bytes are in flight per CU.  ROWS: the longest
// slice the LDS staging of x holds.
// MF: the multiply-adds on the matrix cores instead of the VALU (groups of
// 5-8 batch rows).  Each 16-byte weight load (4 rows x 64 columns per wave)
// feeds four v_mfma_f32_16x16x4_f32: lane l holds W[row l / 16][4 (l % 16)
// + e], the A operand (m = column, k = row) of MFMA e, and x[l % 16][row
// l / 16] from LDS is the B operand (n = batch row), so MFMA e sums the
// lane group's 4 rows for columns 4 i + e.  The VALU form costs 4 B FMAs per
// load, 32 at B = 8 with packed f32 off; the MFMA form 4 MFMAs at any B.
// XS: x is not staged for the whole slice before the loop but streamed with
// the weights: with each step's weight loads a wave loads that step's
// kStep rows of x (lane l: batch row l / 8, rows 4 (l % 8) .. + 3, one
// 16-byte load) and passes them to its lanes through its own two LDS buffers
// (no workgroup barrier: a wave's LDS accesses complete in issue order).
// Needs p.xvec and p.off32.  The staged form's up-front wait for B x K floats per
// workgroup (128 KB at B = 8, K = 4096) goes away.
template <int MAXB, int U, bool VEC, int NW = kWaves, int ROWS = f32_max_rows<MAXB>(), bool MF = false,
          bool XS = false>
__global__ __launch_bounds__(64 * NW) void gemv_f32_kernel(GemvParams p) {
    static_assert(!MF || (VEC && MAXB <= 16), "matrix-core form: 16-byte loads, at most 16 batch rows");
    static_assert(!XS || (VEC && MAXB <= 8 && U == 8),
                  "streamed x: 16-byte loads (W under 4 GB), one x quad per lane and step");
    constexpr int NT = 64 * NW;               // threads
    constexpr int EPL = 4;                    // floats per lane per load
    constexpr int SCOLS = kStripBytes / 4;    // strip columns
    constexpr int kStep = 4 * U;              // rows per wave step
    constexpr int kMaxRows = ROWS;
    // XS buffers: [row][batch] for the VALU form; [batch][row] with a
    // 36-float batch stride for the matrix-core form, whose 64 lanes (batch
    // row l % 16, row l / 16) then read 64 distinct banks.
    constexpr int kXsStride = 36;
    constexpr int kXsBuf = MF ? kXsStride * MAXB : kStep * MAXB;
    constexpr int kRStride = (XS && MF) ? 1 : MAXB;          // floats between rows
    constexpr int kBStride = (XS && MF) ? kXsStride : 1;     // floats between batch rows
    // Staged: this slice's x, [row][batch].  XS: two step buffers per wave.
    __shared__ __attribute__((aligned(16))) float xs[XS ? NW * 2 * kXsBuf : kMaxRows * MAXB];
    __shared__ float red[NW][MAXB][SCOLS];
    __shared__ int last_flag;

    const float *__restrict__ W = static_cast<const float *>(p.w);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t strip = blockIdx.x % p.nstrips;
    const int64_t slice = blockIdx.x / p.nstrips;
    const int64_t col0 = strip * SCOLS;
    const int64_t col = col0 + (lane & 15) * EPL;
    const int rsub = lane >> 4;
    const int64_t nb = p.b < MAXB ? p.b : MAXB;
    const int64_t s_lo = slice * p.kslice;
    const int rows = (int)min(p.kslice, p.k - s_lo);
    if (rows <= 0) {  // K == 0: y = 0, and no row may be read
        store_strip<MAXB, SCOLS, NT, true>(p, strip, slice, nb, col0, &last_flag, [](int, int) { return 0.f; });
        return;
    }
    const int rows_s = (rows + kStep - 1) / kStep * kStep;

    // Activations first, from clamped in-range indices: loads complete in
    // issue order, so the staging below waits only for these while the
    // first weight batch (issued next) streams in behind them.
    // With p.xvec (rows a multiple of 4, x rows 16-byte aligned) each
    // thread loads 4 consecutive rows of one batch row per instruction.
    constexpr int kRowsPerThread = kMaxRows / NT;
    constexpr int kQuads = (kMaxRows / 4 + NT - 1) / NT;  // 4-row groups per thread
    const bool xvec = p.xvec != 0;
    float xv[kRowsPerThread][MAXB];
    f32x4 xq[kQuads][MAXB];
    if constexpr (XS) {
    } else if (xvec) {
#pragma unroll
        for (int i = 0; i < kQuads; ++i) {
            const int qd = min((int)threadIdx.x + NT * i, rows / 4 - 1);
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi)
                xq[i][bi] = *reinterpret_cast<const f32x4 *>(p.x + min<int64_t>(bi, nb - 1) * p.k + s_lo + 4 * qd);
        }
    } else {
#pragma unroll
        for (int i = 0; i < kRowsPerThread; ++i) {
            const int rr = min((int)threadIdx.x + NT * i, rows - 1);
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi) xv[i][bi] = p.x[min<int64_t>(bi, nb - 1) * p.k + s_lo + rr];
        }
    }

    // Each wave walks whole steps of its quarter of the slice.  Loads are
    // unconditional: rows past the slice read its last row (their x is
    // zero); with VEC (N % 4 == 0, aligned W) a lane's 4 columns lie all
    // inside N or all outside it, and lanes past N read the strip's first
    // columns (never stored).  Without VEC every column is checked.
    const int per = ((rows_s / kStep + NW - 1) / NW) * kStep;
    const int wb = min(wave * per, rows_s), we = min(wb + per, rows_s);
    const int64_t lcol = (VEC && col >= p.n) ? col0 : col;
    const float *base = W + s_lo * p.n + lcol;
    // XS (W under 4 GB): addresses as the uniform base plus a 32-bit byte
    // offset per lane, one multiply per step and an add and a clamp per
    // load, instead of a 64-bit multiply per load: the fewer instructions
    // between a step's loads, the sooner the next step's are issued.
    const uint32_t row_bytes = (uint32_t)p.n * 4u;
    const uint32_t lane_off = XS ? (uint32_t)((s_lo * p.n + lcol) * 4) : 0u;
    const uint32_t last_off = lane_off + (uint32_t)(rows - 1) * row_bytes;  // this lane's 16 bytes of the last row
    const char *const wbytes = reinterpret_cast<const char *>(W);
    auto load_step = [&](int r0, i32x4 (&w)[U]) {
        if constexpr (XS) {
            const uint32_t o = lane_off + (uint32_t)(r0 + rsub) * row_bytes;
#pragma unroll
            for (int u = 0; u < U; ++u)
                w[u] = __builtin_nontemporal_load(
                    reinterpret_cast<const i32x4 *>(wbytes + min(o + (uint32_t)(4 * u) * row_bytes, last_off)));
            return;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = max(min(r0 + 4 * u + rsub, rows - 1), 0);
            const float *src = base + (int64_t)r * p.n;
            if constexpr (VEC) {
                w[u] = *reinterpret_cast<const i32x4 *>(src);
            } else {
                float tmp[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) tmp[e] = (col + e < p.n) ? src[e] : 0.f;
                __builtin_memcpy(&w[u], tmp, 16);
            }
        }
    };
    // XS: this lane's x quad of step r0, loaded from a clamped in-range
    // address, and its store into the wave's buffer, zero for rows past the
    // slice and batch rows past nb (rows % 4 == 0 with p.xvec, so a quad is
    // all in or all out).  The mask is applied at the store: a use of the
    // loaded value right after the load made the compiler wait for it there.
    const int xb_row = lane >> 3, xq_off = 4 * (lane & 7);
    const float *xsrc = p.x + min<int64_t>(xb_row, nb - 1) * p.k + s_lo;
    auto load_x = [&](int r0) { return *reinterpret_cast<const f32x4 *>(xsrc + min(r0 + xq_off, rows - 4)); };
    float *const xwave = xs + (XS ? wave * 2 * kXsBuf : 0);
    auto put_x = [&](f32x4 v, int buf, int r0) {
        const uint32_t keep = (r0 + xq_off < rows && xb_row < nb) ? 0xffffffffu : 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float e = v[q];  // (a bit_cast of the element lvalue itself reads element 0)
            v[q] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, e) & keep);
        }
        if (xb_row < MAXB) {
            float *d = xwave + buf * kXsBuf;
            if constexpr (MF) {
                *reinterpret_cast<f32x4 *>(d + xb_row * kXsStride + xq_off) = v;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) d[(xq_off + q) * MAXB + xb_row] = v[q];
            }
        }
        // The other lanes of this wave read what was just written; a
        // wave's LDS accesses complete in issue order.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    __builtin_amdgcn_sched_barrier(0);
    i32x4 wa[U], wn[U];
    f32x4 xa, xn;
    if constexpr (XS) xa = load_x(wb);
    load_step(wb, wa);
    __builtin_amdgcn_sched_barrier(0);

    // Stage x, zero past the slice and the batch (a mask, not a select: a
    // value used only under a condition lets the compiler sink its load into
    // a branch, which then waits for everything issued before it).
    if constexpr (XS) {
    } else if (xvec) {
#pragma unroll
        for (int i = 0; i < kQuads; ++i) {
            const int qd = threadIdx.x + NT * i;
            if (4 * qd >= rows_s) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int bi = 0; bi < MAXB; ++bi) {
                    const uint32_t keep = (4 * qd + q < rows && bi < nb) ? 0xffffffffu : 0u;
                    const float v = xq[i][bi][q];
                    xs[(4 * qd + q) * MAXB + bi] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & keep);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < kRowsPerThread; ++i) {
            const int r = threadIdx.x + NT * i;
            if (r >= rows_s) continue;
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi) {
                const uint32_t keep = (r < rows && bi < nb) ? 0xffffffffu : 0u;
                xs[r * MAXB + bi] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, xv[i][bi]) & keep);
            }
        }
    }
    if constexpr (!XS) __syncthreads();

    float acc[MF ? 1 : MAXB][EPL];
#pragma unroll
    for (int bi = 0; bi < (MF ? 1 : MAXB); ++bi)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[bi][e] = 0.f;
    f32x4 macc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) macc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int bq = lane & 15;  // MF: this lane's batch row (B operand column)
    // xr: x of the row, batch row bi at xr[bi * kBStride].
    auto fma_row = [&](const i32x4 &wv, const float *xr) {
        const f32x4 wf = __builtin_bit_cast(f32x4, wv);
        if constexpr (MF) {
            const float xb = bq < MAXB ? xr[(bq < MAXB ? bq : 0) * kBStride] : 0.f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) macc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(wf[e], xb, macc[e], 0, 0, 0);
        } else {
            float x[MAXB];
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi) x[bi] = xr[bi * kBStride];
#pragma unroll
            for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[bi][e] = fmaf(x[bi], wf[e], acc[bi][e]);  // explicit FMA
        }
    };
    // The next step is requested before the current one is used.  Every
    // branch is wave-uniform and every block issues its loads
    // unconditionally, so the wait for a step never covers the next one.
    // Rows of step r0 from x rows xrow0 on: the staged slice (XS: the buffer).
    auto fma_step = [&](const i32x4 (&w)[U], const float *xbase, int xrow0) {
#pragma unroll
        for (int u = 0; u < U; ++u) fma_row(w[u], xbase + (xrow0 + 4 * u + rsub) * kRStride);
    };
    if constexpr (XS) {
        // x of a step is requested before its weights, with the next step's
        // loads in flight before the current step is used.
        for (int r0 = wb; r0 < we;) {
            if (r0 + kStep >= we) {
                put_x(xa, 0, r0);
                fma_step(wa, xwave, 0);
                break;
            }
            xn = load_x(r0 + kStep);
            load_step(r0 + kStep, wn);
            put_x(xa, 0, r0);
            fma_step(wa, xwave, 0);
            r0 += kStep;
            if (r0 + kStep >= we) {
                put_x(xn, 1, r0);
                fma_step(wn, xwave + kXsBuf, 0);
                break;
            }
            xa = load_x(r0 + kStep);
            load_step(r0 + kStep, wa);
            put_x(xn, 1, r0);
            fma_step(wn, xwave + kXsBuf, 0);
            r0 += kStep;
        }
    } else {
        for (int r0 = wb; r0 < we;) {
            if (r0 + kStep >= we) {
                fma_step(wa, xs, r0);
                break;
            }
            load_step(r0 + kStep, wn);
            fma_step(wa, xs, r0);
            r0 += kStep;
            if (r0 + kStep >= we) {
                fma_step(wn, xs, r0);
                break;
            }
            load_step(r0 + kStep, wa);
            fma_step(wn, xs, r0);
            r0 += kStep;
        }
    }

    if constexpr (MF) {
        // Lane l, register g of MFMA e: column 16 (l / 16) + 4 g + e of the
        // strip, batch row l % 16 (its 4 rows already summed by the MFMA).
        if (bq < MAXB) {
#pragma unroll
            for (int e = 0; e < EPL; ++e)
#pragma unroll
                for (int g = 0; g < 4; ++g) red[wave][bq][16 * (lane >> 4) + 4 * g + e] = macc[e][g];
        }
    } else {
        // Reduce over the 4 row lanes of each column group (lanes l, l ^ 16,
        // l ^ 32, l ^ 48: lane swaps, (l + (l ^ 16)) + ((l ^ 32) + (l ^ 48))),
        // then over waves.
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi)
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float v = quarter_sum(acc[bi][e]);
                if (lane < 16) red[wave][bi][lane * EPL + e] = v;
            }
    }
    __syncthreads();
    auto strip_value = [&](int bi, int c) {
        float v = red[0][bi][c];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) v = v + red[w2][bi][c];
        return v;
    };
    store_strip<MAXB, SCOLS, NT, true>(p, strip, slice, nb, col0, &last_flag, strip_value);
}

// ---- int8 weights on the matrix cores -------------------------------------------
//
// y[b,n] = sum_k xs[b,k] * (q[k,n] - zp[k]) with xs = x * s[k] runs as
// v_mfma_f32_16x16x32_f16 with W as the A operand (m = column, k = row) and
// the split activations as B (k = row, n = split column):
//  * A: lane l holds 8 consecutive rows of one column.  Lane (g = l/16,
//    c = l%16) loads rows 8g..8g+7 of a 32-row block, 16 bytes each
//    (columns 16c..16c+15 of the 256-byte strip), so every load instruction
//    still reads 4 rows x 256 contiguous bytes.  Column 16c + j of those 8
//    rows is then the A operand of MFMA j.
//  * int8 -> f16 is exact and cheap: with u = q ^ 0x80 (= q + 128 as an
//    unsigned byte) the f16 with bits 0x64uu is 1024 + u = 1152 + q, built by
//    two byte permutes per pair of weights; one packed f16 add of
//    -(1152 + zp) per pair of rows leaves q - zp, exact (|q - zp| <= 255).
//  * B: each workgroup scales its slice of xs by a power of two 2^e so that
//    max |xs| 2^e lies in [2^14, 2^15), then splits it into three f16, hi =
//    f16(X), mid = f16(X - hi), lo = f16(X - hi - mid) with X = xs 2^e (each
//    difference exact in fp32): hi + mid + lo carries 33 significant bits,
//    more than X's own 24, so X is carried exactly unless its last bits fall
//    below f16's subnormal step (|X| < 2^-1, i.e. below 2^-16 of the slice
//    maximum), and hi * w, mid * w, lo * w are exact products in the fp32
//    accumulators.  Up to 4 batch rows the three pieces of batch row b sit
//    in split columns b, MAXB + b and 2 MAXB + b of one MFMA; 8 batch rows
//    take two MFMAs per weight fragment, hi / mid in columns b / 8 + b of
//    the first and lo in column b of the second.
// Sums are fp32 in a fixed order, as in the VALU form; the result is within
// the fp32 GEMM bound of the reference, not bit-identical to it.
namespace w8mf {

constexpr int kBlockRows = 32;           // rows per MFMA step of a wave
constexpr int kXStride = kMaxSlice + 8;  // f16 per split column: +16 bytes keeps B reads conflict-free
// B operands (16 split columns each) per weight fragment
template <int MAXB>
constexpr int nbops() { return MAXB <= 4 ? 1 : 2; }
template <int MAXB>
constexpr int xbytes() { return 16 * nbops<MAXB>() * kXStride * 2; }
// Wave partials [wave][batch][column], aliased onto the split activations:
// 2 words of padding per 64 columns and a 264-word row put the 32 lanes
// that store together on 32 distinct banks.
constexpr int kRedStride = 264;
template <int NW, int MAXB>
constexpr int lds_bytes() {
    return xbytes<MAXB>() > NW * 8 * kRedStride * 4 ? xbytes<MAXB>() : NW * 8 * kRedStride * 4;
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int red_index(int w, int b, int col) { return (w * 8 + b) * kRedStride + col + 2 * (col >> 6); }

template <int MAXB, bool VEC, int NW>
__global__ __launch_bounds__(64 * NW, (VEC && NW == 4 && MAXB <= 4) ? 2 : 1) void gemv_w8_mfma_kernel(GemvParams p) {
    constexpr int SCOLS = kStripBytes;
    constexpr int NT = 64 * NW;
    constexpr int NBO = nbops<MAXB>();
    // split column of piece 0 / 1 / 2 (hi / mid / lo) of batch row b
    constexpr int kMidCol = NBO == 1 ? MAXB : 8, kLoCol = NBO == 1 ? 2 * MAXB : 16;
    __shared__ __attribute__((aligned(16))) unsigned char lds[lds_bytes<NW, MAXB>()];
    __shared__ __attribute__((aligned(16))) uint32_t zph[kMaxSlice / 2];  // -(1152 + zp) of row pairs, f16x2
    __shared__ float amax_red[NW];
    __shared__ int last_flag;
    _Float16 *xsh = reinterpret_cast<_Float16 *>(lds);

    const int8_t *__restrict__ W = static_cast<const int8_t *>(p.w);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int64_t strip = blockIdx.x % p.nstrips;
    const int64_t slice = blockIdx.x / p.nstrips;
    const int64_t col0 = strip * SCOLS;
    const int64_t nb = p.b < MAXB ? p.b : MAXB;
    const int64_t s_lo = slice * p.kslice;
    const int rows = (int)min(p.kslice, p.k - s_lo);
    const int rows32 = (rows + kBlockRows - 1) & ~(kBlockRows - 1);
    if (rows <= 0) {  // K == 0: y = 0, and no row may be read
        store_strip<MAXB, SCOLS, NT>(p, strip, slice, nb, col0, &last_flag, [](int, int) { return 0.f; });
        return;
    }

    // Activations first: loads complete in issue order, so the staging below
    // waits only for these, while the first weight blocks (issued next)
    // stream in behind them.  Each thread owns rows threadIdx.x + 256 i.
    // The loads are unconditional, from clamped in-range indices, and the
    // values are selected afterwards: a load under a lane condition would be
    // waited for before the branches rejoin, one memory latency per load.
    constexpr int kRowsPerThread = kMaxSlice / NT;
    float xv[kRowsPerThread][MAXB], sv[kRowsPerThread];
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i) {
        const int rr = min((int)threadIdx.x + NT * i, rows - 1);
        sv[i] = p.scales[s_lo + rr];
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) xv[i][bi] = p.x[min<int64_t>(bi, nb - 1) * p.k + s_lo + rr];
    }
    // Zero points of row pairs threadIdx.x + 256 u.  Without zero points
    // the (ignored) bytes come from the scales, so that no branch guards
    // these loads either.
    constexpr int kPairsPerThread = kMaxSlice / 2 / NT;
    const int8_t *zsrc = p.zps ? p.zps : reinterpret_cast<const int8_t *>(p.scales);
    int zr[kPairsPerThread][2];
#pragma unroll
    for (int u = 0; u < kPairsPerThread; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h) zr[u][h] = zsrc[s_lo + min(2 * ((int)threadIdx.x + NT * u) + h, rows - 1)];

    // Blocks of 32 rows go to the waves round-robin (wave w takes blocks w,
    // w + NW, ...): a read-only probe of this pattern streamed the
    // [4096, 14336] weight in 11.6 us against 12.8 us with contiguous row
    // ranges per wave, whose waves also finished further apart.
    const int nblk = rows32 / kBlockRows;
    const int cnt = wave < nblk ? (nblk - wave + NW - 1) / NW : 0;
    // First row of the wave's i-th block; past the last block it repeats
    // that block (a wave without blocks gets rows that the loads clamp).
    auto block_row = [&](int i) { return (wave + NW * min(i, max(cnt - 1, 0))) * kBlockRows; };
    const int64_t col = col0 + 16 * c;
    // Loads are unconditional so that the wait for a block never has to wait
    // for the prefetch of the next one.  Rows past the slice read its last
    // row (their activations are zero); with VEC (N % 16 == 0, aligned W) a
    // lane's 16 columns lie all inside N or all outside it, and lanes past
    // N read the strip's first columns (never stored).  Without VEC every
    // byte is checked.
    const int64_t lcol = (VEC && col >= p.n) ? col0 : col;
    const int8_t *base = W + s_lo * p.n + lcol;
    auto load_block = [&](int r0, i32x4 (&R)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = max(min(r0 + 8 * g + i, rows - 1), 0);  // row within the slice
            const int8_t *src = base + (int64_t)r * p.n;
            if constexpr (VEC) {
                R[i] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(src));
            } else {
                int8_t tmp[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) tmp[e] = (col + e < p.n) ? src[e] : int8_t(0);
                __builtin_memcpy(&R[i], tmp, 16);
            }
        }
    };
    // The wave's first kBufs blocks are requested before the staging.
    // Unconditional as well (past the wave's blocks they re-read its last
    // block): a branch here would make the staging below wait for these
    // loads.  The scheduling barriers keep the issue order: activations,
    // weights, then the staging arithmetic.  Measured at [4096, 14336] and
    // 1024-row slices, 3 or 4 buffers were no faster than 2 with 4 waves and
    // 1-2 us slower with 8; waiting for the activations before requesting
    // any weights changed nothing either.
    constexpr int kBufs = 2;
    __builtin_amdgcn_sched_barrier(0);
    i32x4 R[kBufs][8];
#pragma unroll
    for (int j = 0; j < kBufs; ++j) load_block(block_row(j), R[j]);
    __builtin_amdgcn_sched_barrier(0);

    // Masks rather than selects: a value that is only used under a
    // condition lets the compiler sink its load into a branch again.
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i) {
        const int r = threadIdx.x + NT * i;
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) {
            const uint32_t keep = (r < rows && bi < nb) ? 0xffffffffu : 0u;
            xv[i][bi] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, xv[i][bi] * sv[i]) & keep);
        }
    }
#pragma unroll
    for (int u = 0; u < kPairsPerThread; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            zr[u][h] &= (p.zps && 2 * ((int)threadIdx.x + NT * u) + h < rows) ? -1 : 0;

    // Stage: power-of-two prescale, f16 hi/lo split into columns [n][row]
    // (zero past the slice), and the zero-point pairs.  Split columns of
    // batch rows past MAXB are never written: an MFMA output column depends
    // only on its own B column, and those are not stored.
    // The prescale comes from the largest FINITE |x s| of the slice, so that
    // every finite value lands at most at 2^15 (no f16 overflow); an
    // infinite or NaN x s becomes hi = itself, lo = 0 below, and its products
    // give inf / NaN as x * dequantize(W) does in the reference.
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i)
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi)
            amax = fmaxf(amax, __builtin_isfinite(xv[i][bi]) ? fabsf(xv[i][bi]) : 0.f);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (lane == 0) amax_red[wave] = amax;
#pragma unroll
    for (int u = 0; u < kPairsPerThread; ++u) {
        const int pr = (int)threadIdx.x + NT * u;
        if (2 * pr < rows32) {
            const half2 z = {(_Float16)(-(1152 + zr[u][0])), (_Float16)(-(1152 + zr[u][1]))};
            zph[pr] = __builtin_bit_cast(uint32_t, z);
        }
    }
    __syncthreads();
    amax = amax_red[0];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) amax = fmaxf(amax, amax_red[w2]);
    int ex = 0;
    if (amax > 0.f) {
        (void)frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1)
        ex = 15 - ex;
    }
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i) {
        const int r = threadIdx.x + NT * i;
        if (r >= rows32) continue;
#pragma unroll
        for (int bi = 0; bi < MAXB; ++bi) {
            const float X = ldexpf(xv[i][bi], ex);
            const _Float16 hi = (_Float16)X;
            const bool fin = __builtin_isfinite(X);
            const float r1 = fin ? X - (float)hi : 0.f;
            const _Float16 mid = (_Float16)r1;
            const _Float16 lo = (_Float16)(r1 - (float)mid);
            xsh[bi * kXStride + r] = hi;
            xsh[(kMidCol + bi) * kXStride + r] = mid;
            xsh[(kLoCol + bi) * kXStride + r] = lo;
        }
    }
    __syncthreads();

    // Stream the weights in 32-row blocks, kBufs blocks in flight.
    f32x4 acc[NBO][16];
#pragma unroll
    for (int o = 0; o < NBO; ++o)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[o][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute_block = [&](const i32x4 (&R)[8], int r0) {
        half8 bx[NBO];
#pragma unroll
        for (int o = 0; o < NBO; ++o)
            bx[o] = *reinterpret_cast<const half8 *>(xsh + (16 * o + c) * kXStride + r0 + 8 * g);
        const u32x4 zq = *reinterpret_cast<const u32x4 *>(zph + (r0 + 8 * g) / 2);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            u32x4 a[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo_r = (uint32_t)R[2 * i][d] ^ 0x80808080u;
                const uint32_t hi_r = (uint32_t)R[2 * i + 1][d] ^ 0x80808080u;
                const uint32_t t0 = __builtin_amdgcn_perm(hi_r, lo_r, 0x05010400u);  // columns 4d, 4d+1
                const uint32_t t1 = __builtin_amdgcn_perm(hi_r, lo_r, 0x07030602u);  // columns 4d+2, 4d+3
                // (a vector element is copied to a scalar before the bit cast:
                // this compiler casts an element lvalue from the vector start)
                const uint32_t zi = zq[i];
                const half2 z = __builtin_bit_cast(half2, zi);
                a[0][i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, __builtin_amdgcn_perm(t0, 0x64646464u, 0x00050004u)) + z);
                a[1][i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, __builtin_amdgcn_perm(t0, 0x64646464u, 0x00070006u)) + z);
                a[2][i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, __builtin_amdgcn_perm(t1, 0x64646464u, 0x00050004u)) + z);
                a[3][i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, __builtin_amdgcn_perm(t1, 0x64646464u, 0x00070006u)) + z);
            }
#pragma unroll
            for (int o = 0; o < NBO; ++o)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    acc[o][4 * d + jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a[jj]), bx[o],
                                                                                acc[o][4 * d + jj], 0, 0, 0);
        }
    };
    // While more than kBufs blocks remain, a buffer is refilled with the
    // block kBufs ahead as soon as it has been consumed; the refills of the
    // last such pass may re-read the wave's last block (an L2 hit) rather
    // than branch around the loads, since a load under a branch would make
    // the wait for the current block cover it too.  The last kBufs buffers
    // are then consumed without refills (the conditions are wave-uniform and
    // guard no loads).
    int i = 0;
    for (; i + kBufs < cnt; i += kBufs) {
#pragma unroll
        for (int j = 0; j < kBufs; ++j) {
            compute_block(R[j], block_row(i + j));
            load_block(block_row(i + j + kBufs), R[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < kBufs; ++j)
        if (i + j < cnt) compute_block(R[j], block_row(i + j));

    // acc[o][j][i] of lane (g, c) is column 16 (4g + i) + j for split
    // column c of B operand o.  The pieces of batch row c < MAXB meet in
    // lane c of each row of 16, summed (hi + mid) + lo: up to 4 batch rows
    // from lanes c + MAXB and c + 2 MAXB of the same row, 8 batch rows from
    // lane c + 8 and the second operand.  DPP row_ror:r gives lane i the
    // value of lane (i - r) mod 16 of its row (checked on gfx950), so lane
    // c + M is row_ror:(16 - M).
    __syncthreads();  // every wave is done with the split activations
    float *red = reinterpret_cast<float *>(lds);
    constexpr int kRorMid = 0x120 + (16 - kMidCol), kRorLo = 0x120 + (16 - kLoCol) % 16;
    auto from_lane = [](float v, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), decltype(ctrl)::value,
                                                                  0xf, 0xf, false));
    };
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = acc[0][j][i];
            float t;
            if constexpr (NBO == 1) {
                const float vm = from_lane(v, std::integral_constant<int, kRorMid>{});
                const float vl = from_lane(v, std::integral_constant<int, kRorLo>{});
                t = (v + vm) + vl;
            } else {
                const float vm = from_lane(v, std::integral_constant<int, kRorMid>{});
                t = (v + vm) + acc[NBO - 1][j][i];
            }
            if (c < MAXB) red[red_index(wave, c, 16 * (4 * g + i) + j)] = t;
        }
    __syncthreads();
    auto strip_value = [&](int bi, int cc) {
        float s = red[red_index(0, bi, cc)];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) s += red[red_index(w2, bi, cc)];
        return ldexpf(s, -ex);
    };
    store_strip<MAXB, SCOLS, NT>(p, strip, slice, nb, col0, &last_flag, strip_value);
}

// NW = 8 exists only with VEC (the caller never asks for it without).
template <int MAXB, int NW = 4>
void launch(const GemvParams &q, bool vec, hipStream_t s) {
    const dim3 grid((unsigned)(q.nstrips * q.slices)), block(64 * NW);
    if (vec)
        hipLaunchKernelGGL((gemv_w8_mfma_kernel<MAXB, true, NW>), grid, block, 0, s, q);
    else if constexpr (NW == 4)
        hipLaunchKernelGGL((gemv_w8_mfma_kernel<MAXB, false, NW>), grid, block, 0, s, q);
}

}  // namespace w8mf

// 8 batch rows in one slice of up to 4096 rows, one 8-wave workgroup per CU:
// x takes 128 KB of LDS, the wave partials 16 KB.
constexpr int kWideRows8 = 4096;

template <int MAXB>
void launch_f32(const GemvParams &p, bool vec, hipStream_t s) {
    constexpr int U = 8;
    const unsigned nwg = (unsigned)(p.nstrips * p.slices);
    // Matrix cores for groups of 5-8 rows: W [4096, 14336] at 8 rows 46.1 ->
    // 44.6 us; at 4 rows both forms take 42.7 us.
    constexpr bool MF = MAXB >= 8;
    if constexpr (MAXB <= 8) {
        if (vec && p.xvec && p.off32) {  // x streamed with the weights, no staging
            if (nwg <= 256)
                hipLaunchKernelGGL((gemv_f32_kernel<MAXB, U, true, 8, f32_max_rows<MAXB>(), MF, true>), dim3(nwg),
                                   dim3(512), 0, s, p);
            else
                hipLaunchKernelGGL((gemv_f32_kernel<MAXB, U, true, kWaves, f32_max_rows<MAXB>(), MF, true>),
                                   dim3(nwg), dim3(kThreads), 0, s, p);
            return;
        }
    }
    if constexpr (MAXB == 8) {
        if (vec && nwg <= 256 && p.kslice > f32_max_rows<8>()) {
            hipLaunchKernelGGL((gemv_f32_kernel<8, U, true, 8, kWideRows8, MF>), dim3(nwg), dim3(512), 0, s, p);
            return;
        }
    }
    if (vec && nwg <= 256)
        hipLaunchKernelGGL((gemv_f32_kernel<MAXB, U, true, 8, f32_max_rows<MAXB>(), MF>), dim3(nwg), dim3(512), 0, s,
                           p);
    else if (vec)
        hipLaunchKernelGGL((gemv_f32_kernel<MAXB, U, true, kWaves, f32_max_rows<MAXB>(), MF>), dim3(nwg),
                           dim3(kThreads), 0, s, p);
    else if constexpr (MAXB <= 8)
        hipLaunchKernelGGL((gemv_f32_kernel<MAXB, U, false>), dim3(nwg), dim3(kThreads), 0, s, p);
}

// Rows per K-slice of the int8 MFMA kernel: the longest slice, up to
// kMaxSlice, that still gives at least 192 workgroups.  Its fixed cost per
// workgroup (staging the activations, reducing the waves, publishing the
// partial) favours long slices: at [4096, 14336] 1024 rows measured
// 17-19 us for 1-8 batch rows against 18-21 us at 512 and 26-41 us at 128.
int64_t choose_kslice_w8(int64_t nstrips, int64_t k) {
    int64_t ks = kMaxSlice;
    while (ks > 128 && nstrips * ((k + ks - 1) / ks) < 192) ks /= 2;
    return ks;
}

// Rows per K-slice of the fp32 kernel.  All of K in one slice (up to
// f32_max_rows) when the strips alone give at least 192 workgroups: no
// partial strips, no arrival count, no last-arriver sum.  Measured at
// W [4096, 14336] (224 strips), 1 batch row: 41.5 us in one slice against
// 44.1 / 46.1 / 46.7 us in 2 / 4 / 8.  Otherwise 512 rows, halved while
// there would be fewer than ~448 workgroups (each CU streams only ~30-45
// GB/s, so all CUs must take part), at least 128 rows, a multiple of 128 --
// and enlarged so the partial strips written and read back stay under ~10%
// of the weight bytes (5% for groups of 8 batch rows), up to max_rows.
int64_t choose_kslice_f32(int64_t nstrips, int64_t k, int64_t nb, int64_t max_rows) {
    if (nstrips >= 192 && k <= max_rows) return k;
    int64_t ks = 512;
    while (ks > 128 && nstrips * ((k + ks - 1) / ks) < 448) ks /= 2;
    const double cap = nb >= 8 ? 0.05 : 0.10;
    const int64_t max_slices = (int64_t)(cap * (double)k * 4.0 / (8.0 * (double)nb));
    if (max_slices >= 1) ks = std::max(ks, (k + max_slices - 1) / max_slices);
    else ks = k;
    ks = (ks + 127) & ~(int64_t)127;
    return std::min<int64_t>(ks, max_rows);
}

// Where the split-K partial strips and arrival counters of a call live:
// either the per-stream buffers the library allocates on demand (fixed ==
// false), or a fixed region that the allocation-free entry point owns.
struct SplitScratch {
    bool fixed = false;
    float *part = nullptr;
    size_t part_bytes = 0;
    int *counters = nullptr;
    size_t ncounters = 0;
};

// Sets the slicing of one batch group and, for more than one slice, its
// partial workspace and arrival counters.  Groups of a call run one after
// another on the stream, so they share the workspace.
int set_slices(GemvParams &q, int64_t kslice, hipStream_t s, const SplitScratch &sc) {
    q.kslice = kslice;
    q.slices = q.k > 0 ? (q.k + kslice - 1) / kslice : 1;
    q.part = nullptr;
    q.counters = nullptr;
    if (q.slices > 1) {
        const size_t part_bytes = sizeof(float) * (size_t)(q.slices * q.b * q.n);
        if (sc.fixed) {
            if (part_bytes > sc.part_bytes || (size_t)q.nstrips > sc.ncounters)
                return set_error(GFH_INVALID_SHAPE, "gemv_w8: %zu bytes of partials and %lld counters exceed the "
                                 "fixed scratch (%zu bytes, %zu counters)", part_bytes, (long long)q.nstrips,
                                 sc.part_bytes, sc.ncounters);
            q.part = sc.part;
            q.counters = sc.counters;
            return GFH_SUCCESS;
        }
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, part_bytes, &ws));
        q.part = static_cast<float *>(ws);
        GFH_TRY(stream_counters(s, (size_t)q.nstrips, &q.counters));
    }
    return GFH_SUCCESS;
}

// The batch is processed in groups of at most `group` rows.
template <typename F>
int for_batch_groups(const GemvParams &p, const float *x, float *y, int64_t b, F launch_group, int64_t group = 8) {
    for (int64_t b0 = 0; b0 < b; b0 += group) {
        GemvParams q = p;
        q.x = x + b0 * p.k;
        q.y = y + b0 * p.n;
        q.b = (b - b0) < group ? (b - b0) : group;
        GFH_TRY(launch_group(q));
    }
    return GFH_SUCCESS;
}

}  // namespace

int launch_gemv_f32(const float *x, const float *w, float *y, int64_t b, int64_t k, int64_t n, hipStream_t s) {
    return launch_gemv_f32_epi(x, w, y, b, k, n, 1.f, 0.f, nullptr, s);
}

int launch_gemv_f32_epi(const float *x, const float *w, float *y, int64_t b, int64_t k, int64_t n, float alpha,
                        float beta, const float *bias, hipStream_t s) {
    GemvParams p{};
    p.alpha = alpha;
    p.beta = beta;
    p.bias = bias;
    p.epi = alpha != 1.f || beta != 0.f || bias != nullptr;
    p.w = w;
    p.k = k;
    p.n = n;
    p.nstrips = (n + kStripBytes / 4 - 1) / (kStripBytes / 4);
    const bool vec = n % 4 == 0 && aligned16(w);
    p.xvec = (k % 4 == 0) && aligned16(x);
    // (64 rows of margin: a step's offsets are formed before the clamp to the last row)
    p.off32 = ((double)k + 64.0) * (double)n * 4.0 < 4294967296.0;
    // 9-16 rows on the matrix cores in one launch (a 16-column B operand)
    const int64_t group = (b > 8 && vec) ? 16 : 8;
    return for_batch_groups(p, x, y, b, [&](GemvParams &q) {
        const int maxb = q.b == 1 ? 1 : q.b == 2 ? 2 : q.b <= 4 ? 4 : q.b <= 8 ? 8 : 16;
        int64_t max_rows = maxb == 1   ? f32_max_rows<1>()
                           : maxb == 2 ? f32_max_rows<2>()
                           : maxb == 4 ? f32_max_rows<4>()
                           : maxb == 8 ? f32_max_rows<8>()
                                       : f32_max_rows<16>();
        // 8 batch rows: all of K <= 4096 in one slice when the strips alone
        // fill the GPU with one 8-wave workgroup per CU (W [4096, 14336]:
        // see kWideRows8), instead of 4 slices of 1024 rows.
        if (maxb == 8 && vec && k > 0 && k <= kWideRows8 && q.nstrips >= 192 && q.nstrips <= 256)
            max_rows = kWideRows8;
        GFH_TRY(set_slices(q, k > 0 ? choose_kslice_f32(q.nstrips, k, q.b, max_rows) : 32, s, SplitScratch{}));
        if (maxb == 1)
            launch_f32<1>(q, vec, s);
        else if (maxb == 2)
            launch_f32<2>(q, vec, s);
        else if (maxb == 4)
            launch_f32<4>(q, vec, s);
        else if (maxb == 8)
            launch_f32<8>(q, vec, s);
        else
            launch_f32<16>(q, vec, s);
        return check_launch("gemv_f32");
    }, group);
}

namespace {

int gemv_w8_common(const float *x, const int8_t *qw, const float *scales, const int8_t *zps, float *y, int64_t b,
                   int64_t k, int64_t n, hipStream_t s, const SplitScratch &sc) {
    GemvParams p{};
    p.w = qw;
    p.scales = scales;
    p.zps = zps;
    p.k = k;
    p.n = n;
    p.nstrips = (n + kStripBytes - 1) / kStripBytes;
    const bool vec = n % 16 == 0 && aligned16(qw);
    return for_batch_groups(p, x, y, b, [&](GemvParams &q) {
        GFH_TRY(set_slices(q, k > 0 ? choose_kslice_w8(q.nstrips, k) : 128, s, sc));
        // At most one workgroup per CU: 8 waves each, so that twice the weight
        // blocks are in flight while the activations are staged (at
        // [4096, 14336] and 1024-row slices, 1-8 batch rows: 16.6-18.2 us
        // against 17.0-19.4 with 4 waves; with two workgroups per CU, 4
        // waves are faster).
        // (Without VEC, 8 waves would spill registers.)
        const bool wide = vec && q.nstrips * q.slices <= 256;
        auto go = [&](auto maxb) {
            constexpr int MB = decltype(maxb)::value;
            // 8 batch rows carry two accumulator sets (the activations'
            // three pieces take 24 split columns): 4 waves with a whole SIMD
            // each (19.5 us at [4096, 14336]), where 8 waves spill (8 waves
            // with one block in flight: 20.3 us; 4 waves with 3 or 4 blocks in
            // flight: 20.1 / 20.4 us).
            if constexpr (MB <= 4) {
                if (wide)
                    w8mf::launch<MB, 8>(q, vec, s);
                else
                    w8mf::launch<MB, 4>(q, vec, s);
            } else {
                w8mf::launch<MB, 4>(q, vec, s);
            }
        };
        if (q.b == 1)
            go(std::integral_constant<int, 1>{});
        else if (q.b == 2)
            go(std::integral_constant<int, 2>{});
        else if (q.b <= 4)
            go(std::integral_constant<int, 4>{});
        else
            go(std::integral_constant<int, 8>{});
        return check_launch("gemv_w8");
    });
}

// ---- the allocation-free variant ---------------------------------------------
//
// Its split-K partials and arrival counters live in `scratch`, a static
// device array (each GPU the library runs on holds its own copy, at its own
// address, until the process ends).  Host code never uses the array's name
// as an address: it keeps the device address hipGetSymbolAddress returns,
// per device, taken on the entry point's first call on that device.
constexpr size_t kNoAllocCounters = 16384;           // arrival counters (int32)
constexpr size_t kNoAllocPartBytes = (size_t)8 << 20;  // split-K partial strips
constexpr size_t kNoAllocBytes = kNoAllocCounters * sizeof(int) + kNoAllocPartBytes;
constexpr int kMaxDevices = 64;

std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kMaxDevices] = {};

__global__ void zero_ints_kernel(int *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

// Device address of this device's copy of `scratch`.
int noalloc_scratch(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return set_error(GFH_COMPUTATION_FAILED, "hipGetDevice failed");
    }
    if (dev < 0 || dev >= kMaxDevices) return set_error(GFH_COMPUTATION_FAILED, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return set_error(GFH_COMPUTATION_FAILED, "hipGetSymbolAddress(scratch) failed: %s",
                             hipGetErrorString(e));
        }
        g_noalloc_ptr[dev] = p;
    }
    *out = g_noalloc_ptr[dev];
    return GFH_SUCCESS;
}

}  // namespace

int launch_gemv_w8(const float *x, const int8_t *qw, const float *scales, const int8_t *zps, float *y, int64_t b,
                   int64_t k, int64_t n, hipStream_t s) {
    return gemv_w8_common(x, qw, scales, zps, y, b, k, n, s, SplitScratch{});
}

int launch_gemv_w8_noalloc(const float *x, const int8_t *qw, const float *scales, const int8_t *zps, float *y,
                           int64_t b, int64_t k, int64_t n, hipStream_t s) {
    // Sizes first: the first batch group (the largest) needs the most, and
    // nothing is launched when it does not fit.
    const int64_t nstrips = (n + kStripBytes - 1) / kStripBytes;
    const int64_t kslice = k > 0 ? choose_kslice_w8(nstrips, k) : 128;
    const int64_t slices = k > 0 ? (k + kslice - 1) / kslice : 1;
    const int64_t b0 = b < 8 ? b : 8;
    if (slices > 1 && ((size_t)nstrips > kNoAllocCounters ||
                       sizeof(float) * (size_t)slices * (size_t)b0 * (size_t)n > kNoAllocPartBytes))
        return set_error(GFH_INVALID_SHAPE,
                         "gemv_w8_noalloc: k=%lld n=%lld needs %lld slices x %lld rows x %lld columns of partials "
                         "and %lld counters; the fixed scratch holds %zu bytes of partials and %zu counters",
                         (long long)k, (long long)n, (long long)slices, (long long)b0, (long long)n,
                         (long long)nstrips, kNoAllocPartBytes, kNoAllocCounters);
    void *base = nullptr;
    GFH_TRY(noalloc_scratch(&base));
    SplitScratch sc;
    sc.fixed = true;
    sc.counters = static_cast<int *>(base);
    sc.ncounters = kNoAllocCounters;
    sc.part = reinterpret_cast<float *>(static_cast<unsigned char *>(base) + kNoAllocCounters * sizeof(int));
    sc.part_bytes = kNoAllocPartBytes;
    if (slices > 1) {
        // The counters must start at zero.  A completed call leaves them at
        // zero, but the array keeps whatever the last call on this GPU left,
        // so they are cleared here, by a kernel (no memset node, so a caller
        // may capture the call in a graph).
        const unsigned grid = (unsigned)std::min<int64_t>((nstrips + 255) / 256, 64);
        hipLaunchKernelGGL(zero_ints_kernel, dim3(grid), dim3(256), 0, s, sc.counters, nstrips);
        GFH_TRY(check_launch("gemv_w8_noalloc (counter clear)"));
    }
    return gemv_w8_common(x, qw, scales, zps, y, b, k, n, s, sc);
}

}  // namespace gfh
