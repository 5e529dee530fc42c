// qgemm.hip -- INT8 linear on CDNA4 i8 MFMA (v_mfma_i32_32x32x32_i8).
//
//   raw[m,n] = sum_k qx[m,k] * qw[n,k]                       (exact int32)
//   acc[m,n] = raw - zx * rowsum[n]                          (exact int32)
//   y[m,n]   = (float)acc * (sx * sw[n]) (+ bias[n])         (f32 roundings)
//
// The reference quantizes with quantization.rs:77-153 and computes the layer
// as dequantize + fp32 matmul (quantization.rs:275-277); the integer form
// above is that layer's int32-accumulate equivalent.  The zero-point term is
// folded out of the inner loop through rowsum[n] = sum_k qw[n,k], so the
// MFMA loop multiplies raw codes only.
//
// Design: one 256-thread workgroup (4 wave64s, 2 x 2) per 128 x 128 output
// tile; each wave holds 2 x 2 32x32 int32 accumulators.  Both operands are
// K-contiguous ([m,k] and [n,k]), so both are staged into LDS as
// [rows][BK + 16] byte tiles (16-byte pad keeps the 16-byte fragment reads
// of 8 consecutive rows on distinct banks) and read with one ds_read_b128
// per lane per MFMA: lane l supplies row l%32 and bytes k0 + 16*(l/32) ..
// +15 for A and the same k range for B, so every product pairs matching k
// (the integer sum is exact in any order).  Two LDS stages, global loads for
// stage t+1 issued before the MFMAs of stage t, one barrier per stage, and
// the same XCD-contiguous / GROUP_M tile order as the fp32 GEMM.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

// Every multiply and add below is its own f32 rounding, as in the reference
// (rustc never contracts a*b+c into an FMA); the MFMA accumulation itself is
// not affected by this pragma.
#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kWM = 64, kWN = 64;
constexpr int kPadB = 16;
constexpr int kStride = kBK + kPadB;  // bytes per LDS row
constexpr int kTileBytes = kBM * kStride;
constexpr int kGroupM = 8;

struct QParams {
    const int8_t *qx;
    const float *sx;
    const int8_t *zx;
    const int8_t *qw;
    const float *sw;
    const int32_t *rowsum;
    const float *bias;
    float *y;
    int32_t *acc;
    int64_t m, n, k;
    int x_per_row;
    int tiles_m, tiles_n;
};

// One 128 x BK byte stage of a K-contiguous int8 operand: 1024 16-byte
// vectors, 4 per thread.
template <bool VEC>
struct I8Stage {
    static constexpr int kVecs = kBM * kBK / 16;
    static constexpr int kPer = kVecs / kThreads;
    i32x4 r[kPer];

    __device__ __forceinline__ void load(const int8_t *__restrict__ base, int64_t row0, int64_t rows_total,
                                         int64_t k0, int64_t k_total, int tid) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int idx = tid + i * kThreads;
            const int64_t row = row0 + idx / (kBK / 16);
            const int64_t kk = k0 + (idx % (kBK / 16)) * 16;
            const int8_t *p = base + row * k_total + kk;
            if (VEC && row < rows_total && kk + 15 < k_total) {
                r[i] = *reinterpret_cast<const i32x4 *>(p);
            } else {
                uint32_t w[4] = {0u, 0u, 0u, 0u};
                if (row < rows_total) {
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (kk + e < k_total) w[e >> 2] |= (uint32_t)(uint8_t)p[e] << (8 * (e & 3));
                }
                r[i] = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            }
        }
    }

    __device__ __forceinline__ void store(int8_t *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int idx = tid + i * kThreads;
            const int row = idx / (kBK / 16);
            const int kb = (idx % (kBK / 16)) * 16;
            *reinterpret_cast<i32x4 *>(lds + row * kStride + kb) = r[i];
        }
    }
};

template <bool VEC>
__global__ __launch_bounds__(kThreads) void qlinear_mfma_kernel(QParams p) {
    constexpr int FM = kWM / 32, FN = kWN / 32;
    __shared__ __attribute__((aligned(16))) int8_t lds[4 * kTileBytes];  // A0 A1 B0 B1
    int8_t *const lds_a = lds;
    int8_t *const lds_b = lds + 2 * kTileBytes;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave >> 1) * kWM;
    const int wn0 = (wave & 1) * kWN;

    const int nblk = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int group_size = kGroupM * p.tiles_n;
    const int group = bid / group_size;
    const int first_m = group * kGroupM;
    const int gm = min(p.tiles_m - first_m, kGroupM);
    const int in_group = bid - group * group_size;
    const int64_t m0 = (int64_t)(first_m + in_group % gm) * kBM;
    const int64_t n0 = (int64_t)(in_group / gm) * kBN;

    i32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    I8Stage<VEC> ga, gb;
    const int64_t nst = (p.k + kBK - 1) / kBK;
    if (nst > 0) {
        ga.load(p.qx, m0, p.m, 0, p.k, tid);
        gb.load(p.qw, n0, p.n, 0, p.k, tid);
        ga.store(lds_a, tid);
        gb.store(lds_b, tid);
    }
    __syncthreads();

    const int frag_row = lane & 31;
    const int frag_k = 16 * (lane >> 5);
    for (int64_t st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) {
            ga.load(p.qx, m0, p.m, (st + 1) * kBK, p.k, tid);
            gb.load(p.qw, n0, p.n, (st + 1) * kBK, p.k, tid);
        }
        const int8_t *la = lds_a + cur * kTileBytes;
        const int8_t *lb = lds_b + cur * kTileBytes;
#pragma unroll
        for (int ks = 0; ks < kBK / 32; ++ks) {
            i32x4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const i32x4 *>(la + (wm0 + i * 32 + frag_row) * kStride + ks * 32 + frag_k);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *reinterpret_cast<const i32x4 *>(lb + (wn0 + j * 32 + frag_row) * kStride + ks * 32 + frag_k);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            ga.store(lds_a + (cur ^ 1) * kTileBytes, tid);
            gb.store(lds_b + (cur ^ 1) * kTileBytes, tid);
        }
        __syncthreads();
    }

    // Epilogue: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn0 + j * 32 + (lane & 31);
        if (col >= p.n) continue;
        const int32_t rs = p.zx ? p.rowsum[col] : 0;
        const float swc = p.y ? p.sw[col] : 0.f;
        const float bc = p.bias ? p.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= p.m) continue;
                const int64_t g = p.x_per_row ? row : 0;
                int32_t a = acc[i][j][r];
                if (p.zx) a = (int32_t)((uint32_t)a - (uint32_t)((int32_t)p.zx[g] * rs));
                if (p.acc) p.acc[row * p.n + col] = a;
                if (p.y) {
                    const float s = p.sx[g] * swc;
                    float v = (float)a * s;
                    if (p.bias) v = v + bc;
                    p.y[row * p.n + col] = v;
                }
            }
        }
    }
}


// ---- large tiles: 256 x 256 per workgroup, direct-to-LDS loads -------------------
//
// For M >= 1024 (compute-bound) each workgroup owns a 256 x 256 output tile
// and each of its 4 waves a 128 x 128 sub-tile: 4 x 4 v_mfma_i32_32x32x32_i8
// accumulators (256 registers per lane), so every 16-byte LDS fragment
// feeds 4 MFMAs and the LDS read rate stays at half the MFMA rate.
// Operands stream through a 4-deep ring of BK = 64 byte stages filled with
// global_load_lds_dwordx4 (global memory straight into LDS, no VGPR
// staging).  Rows of a stage are 64 bytes = 4 chunks of 16; chunk c of row
// r is stored at position c ^ swz(r), which spreads the 16-byte fragment
// reads over distinct banks.  Each lane of a
// load instruction fetches the chunk that lands at its own LDS slot, so the
// swizzle costs nothing on the load side.  Rows past M / N are clamped to
// the last row (their products are never stored); K must be a multiple of 64.
namespace big {

constexpr int kBM = 256, kBN = 256, kBK = 64, kStages = 4;
constexpr int kStageBytes = kBM * kBK;  // one operand, one stage (16 KB)
constexpr int kGroupM = 4;
constexpr int kOutStride = 136;  // floats per row of a wave's output staging area
constexpr int kLdsBytes = (kStages * 2 * kStageBytes > 4 * 64 * kOutStride * 4) ? kStages * 2 * kStageBytes
                                                                                 : 4 * 64 * kOutStride * 4;

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(1))) void *glb_ptr;

// Chunk swizzle of a 64-byte row.  A wave's fragment read has lanes 0-31 on
// rows 0-31 of a block at one logical chunk (lanes 32-63 at the next); with
// chunk ^ ((row >> 2) & 3) those 16-byte reads are conflict-free on gfx950's
// 64-bank LDS (measured: 4.3 clk per ds_read_b128 per CU, against 8.3 for
// chunk ^ ((row >> 1) ^ (row >> 3)) & 3 and 15.8 unswizzled).
__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

// s_waitcnt with only vmcnt constrained (expcnt / lgkmcnt left at maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Waits until at most 8 * n of this wave's stage loads are in flight.
__device__ __forceinline__ void wait_stages(int n) {
    if (n >= 3)
        wait_vmcnt<24>();
    else if (n == 2)
        wait_vmcnt<16>();
    else if (n == 1)
        wait_vmcnt<8>();
    else
        wait_vmcnt<0>();
}

template <bool X_PER_ROW, bool WANT_ACC>
__global__ __launch_bounds__(kThreads, 1) void qlinear_tile256_kernel(QParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[kLdsBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = (wave >> 1) * 128;
    const int wn0 = (wave & 1) * 128;

    const int nblk = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int group_size = kGroupM * p.tiles_n;
    const int group = bid / group_size;
    const int first_m = group * kGroupM;
    const int gm = min(p.tiles_m - first_m, kGroupM);
    const int in_group = bid - group * group_size;
    const int64_t m0 = (int64_t)(first_m + in_group % gm) * kBM;
    const int64_t n0 = (int64_t)(in_group / gm) * kBN;

    // Per-lane source addresses of this wave's 4 A and 4 B load
    // instructions: instruction j covers tile rows wave*64 + 16j .. +15;
    // lane l fills LDS slot l of that 1 KB run (row l/4, physical chunk l%4).
    const int8_t *a_src[4];
    const int8_t *b_src[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = wave * 64 + j * 16 + (lane >> 2);
        const int c = (lane & 3) ^ swz(r);
        a_src[j] = p.qx + min(m0 + r, p.m - 1) * p.k + c * 16;
        b_src[j] = p.qw + min(n0 + r, p.n - 1) * p.k + c * 16;
    }
    const int nk = (int)(p.k / kBK);

    auto issue = [&](int t) {
        int8_t *la = lds + (t % kStages) * 2 * kStageBytes + wave * 64 * kBK;
        int8_t *lb = la + kStageBytes;
        const int64_t k0 = (int64_t)t * kBK;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_global_load_lds((glb_ptr)(a_src[j] + k0), (lds_ptr)(la + j * 16 * kBK), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((glb_ptr)(b_src[j] + k0), (lds_ptr)(lb + j * 16 * kBK), 16, 0, 0);
        }
    };

    // Fragment address inside a stage: lane l reads row l%32 of a 32-row
    // block, logical chunk 2*ks + l/32.
    const int frow = lane & 31;
    const int foff0 = frow * kBK + (((lane >> 5) ^ swz(frow)) * 16);
    const int foff1 = frow * kBK + (((2 + (lane >> 5)) ^ swz(frow)) * 16);

    i32x4 af[2][4], bf[2][4];
    auto load_frags = [&](int buf, int t, int ks) {
        const int8_t *la = lds + (t % kStages) * 2 * kStageBytes;
        const int8_t *lb = la + kStageBytes;
        const int fo = ks ? foff1 : foff0;
#pragma unroll
        for (int i = 0; i < 4; ++i) af[buf][i] = *reinterpret_cast<const i32x4 *>(la + (wm0 + i * 32) * kBK + fo);
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[buf][j] = *reinterpret_cast<const i32x4 *>(lb + (wn0 + j * 32) * kBK + fo);
    };

    i32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    auto mfmas = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[buf][i], bf[buf][j], acc[i][j], 0, 0, 0);
    };

    // Ring of 4 stages, all in flight at once: stage t+4 is issued into
    // stage t's buffer as soon as every wave holds stage t's fragments.
    const int pre = min(kStages, nk);
    for (int t = 0; t < pre; ++t) issue(t);
    wait_stages(pre - 1);
    __builtin_amdgcn_s_barrier();
    load_frags(0, 0, 0);

    for (int t = 0; t < nk; ++t) {
        load_frags(1, t, 1);
        mfmas(0);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();  // this wave's reads of stage t are done
        if (t + 1 < nk) {
            // stage t+1 landed: stages t+2, t+3 may still be in flight
            wait_stages(min(2, nk - t - 2));
            __builtin_amdgcn_s_barrier();
            if (t + kStages < nk) issue(t + kStages);
            load_frags(0, t + 1, 0);
        }
        mfmas(1);
    }

    // Epilogue: lane l, register r of block (i, j) holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32 of that 32 x 32 block.
    // Per-tensor activation parameters are uniform; per-row ones are read
    // once per row.
    const int zx0 = (!X_PER_ROW && p.zx) ? (int)p.zx[0] : 0;
    const float sx0 = (!X_PER_ROW && p.y) ? p.sx[0] : 0.f;
    int32_t rs[4];
    float swc[4], bc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t col = min(n0 + wn0 + j * 32 + (lane & 31), p.n - 1);
        rs[j] = p.zx ? p.rowsum[col] : 0;
        swc[j] = p.y ? p.sw[col] : 0.f;
        bc[j] = p.bias ? p.bias[col] : 0.f;
    }
    // The dequantized value of accumulator register r of block (i, j), and
    // its exact int32 accumulator (zero-point term removed).
    auto finish = [&](int i, int j, int r, int32_t &a) -> float {
        a = acc[i][j][r];
        float sc;
        if (X_PER_ROW) {
            const int64_t row = min(m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), p.m - 1);
            if (p.zx) a = (int32_t)((uint32_t)a - (uint32_t)((int32_t)p.zx[row] * rs[j]));
            sc = p.y ? p.sx[row] * swc[j] : 0.f;
        } else {
            a = (int32_t)((uint32_t)a - (uint32_t)(zx0 * rs[j]));
            sc = sx0 * swc[j];
        }
        float v = (float)a * sc;
        if (p.bias) v = v + bc[j];
        return v;
    };

    if (WANT_ACC) {
        // Parity/debug variant: int32 accumulators and outputs stored
        // straight from registers.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t col = n0 + wn0 + j * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    int32_t a;
                    const float v = finish(i, j, r, a);
                    if (col < p.n && row < p.m) {
                        p.acc[row * p.n + col] = a;
                        if (p.y) p.y[row * p.n + col] = v;
                    }
                }
        }
        return;
    }

    // Output tile through LDS: each wave converts 64 rows x 128 columns at a
    // time into its own region (row stride 136 floats keeps the two row
    // groups of one ds_write_b32 on disjoint banks), then writes whole
    // 512-byte row runs with 16-byte stores.
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();  // every wave is done with the operand ring
    float *lt = reinterpret_cast<float *>(lds) + wave * (64 * kOutStride);
    const bool vec_out = (p.n % 4) == 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    int32_t a;
                    const float v = finish(2 * h + ii, j, r, a);
                    const int lr = ii * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    lt[lr * kOutStride + j * 32 + (lane & 31)] = v;
                }
        // each read covers 2 rows x 128 columns: lane l -> row 2q + l/32,
        // columns 4*(l%32) .. +3
        const int64_t col = n0 + wn0 + 4 * (lane & 31);
#pragma unroll
        for (int q = 0; q < 32; ++q) {
            const int lr = 2 * q + (lane >> 5);
            const f32x4 v = *reinterpret_cast<const f32x4 *>(lt + lr * kOutStride + 4 * (lane & 31));
            const int64_t row = m0 + wm0 + h * 64 + lr;
            if (row >= p.m) continue;
            float *dst = p.y + row * p.n + col;
            if (vec_out && col + 3 < p.n) {
                *reinterpret_cast<f32x4 *>(dst) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < p.n) dst[e] = v[e];
            }
        }
    }
}

}  // namespace big


// ---- skinny M (decode): weights streamed from HBM straight into MFMA ----------
//
// For M <= 64 the layer is HBM-bound (the weight is read once, 45 MB at the
// BASELINE shape).  W [N, K] is K-contiguous, which is exactly the per-lane
// operand layout of v_mfma_i32_16x16x64_i8 (lane l: row / column l % 16,
// 16 consecutive k bytes), so weight fragments are plain 16-byte global
// loads straight into registers, and so are the fragments of x (at most
// 64 x K bytes, cache-resident).
//  * A workgroup owns 16 output columns; its 4 waves split the K range
//    four ways and their exact int32 accumulators are added through LDS at
//    the end, so the waves never wait for one another.
//  * One weight load instruction covers 16 rows x 64 contiguous bytes;
//    kU k-steps per lane are in flight (512 contiguous bytes per row).
//  * With fewer than ~512 column blocks, K is also split over workgroups:
//    each publishes its int32 partial tile with agent-scope stores and
//    counts its arrival; the last one of the column block sums the slices
//    (integer, so exact in any order) and runs the dequantizing epilogue.
namespace skinny {

constexpr int kCols = 16;  // output columns per workgroup
constexpr int kWaves = kThreads / 64;
constexpr int kU = 8;

struct SkParams {
    QParams q;
    int64_t kslice, slices, nblk;
    int32_t *part;  // [slices][m][n] partial accumulators (slices > 1)
    int *counters;  // one per column block, zero at rest (slices > 1)
};

template <int MB>
__global__ __launch_bounds__(kThreads) void qlinear_skinny_kernel(SkParams sp) {
    const QParams &p = sp.q;
    __shared__ i32x4 red[kWaves - 1][MB][64];
    __shared__ int last_flag;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t blk = blockIdx.x % sp.nblk, slice = blockIdx.x / sp.nblk;
    const int64_t n0 = blk * kCols;
    // This wave's k-steps (64 bytes each) inside the slice.
    const int64_t k_lo = slice * sp.kslice;
    const int kl = (int)min(sp.kslice, p.k - k_lo);  // a multiple of 16
    const int nsteps = (kl + 63) / 64;
    const int per = (nsteps + kWaves - 1) / kWaves;
    const int st0 = min(wave * per, nsteps), st1 = min(st0 + per, nsteps);

    // Fragment sources: lane l -> weight row n0 + l % 16 (clamped; such
    // columns are never stored) / x row l % 16 + 16 mb, bytes 16 * (l / 16)
    // of each 64-byte k-step.
    const int kb = 16 * (lane >> 4);
    const int8_t *wsrc = p.qw + min(n0 + (lane & 15), p.n - 1) * p.k + k_lo + kb;
    const int8_t *xsrc = p.qx + k_lo + kb;

    i32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = i32x4{0, 0, 0, 0};
    for (int s0 = st0; s0 < st1; s0 += kU) {
        i32x4 w[kU], xf[kU][MB];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int off = (s0 + u) * 64;
            const bool ok = s0 + u < st1 && off + kb < kl;
            w[u] = ok ? *reinterpret_cast<const i32x4 *>(wsrc + off) : i32x4{0, 0, 0, 0};
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int64_t row = mb * 16 + (lane & 15);
                xf[u][mb] = (ok && row < p.m) ? *reinterpret_cast<const i32x4 *>(xsrc + row * p.k + off)
                                              : i32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xf[u][mb], w[u], acc[mb], 0, 0, 0);
    }

    // Add the four waves' accumulators (exact int32) in wave 0.
    if (wave > 0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) red[wave - 1][mb][lane] = acc[mb];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int w2 = 0; w2 < kWaves - 1; ++w2) acc[mb] += red[w2][mb][lane];

    // 16x16 accumulator layout: lane l, register r -> row 4 * (l / 16) + r,
    // column l % 16 of the block.
    const int64_t col = n0 + (lane & 15);
    const bool col_ok = col < p.n;
    auto row_of = [&](int mb, int r) -> int64_t { return (int64_t)mb * 16 + 4 * (lane >> 4) + r; };
    auto epilogue = [&](int64_t row, int32_t raw) {
        const int64_t g = p.x_per_row ? row : 0;
        int32_t a = raw;
        if (p.zx) a = (int32_t)((uint32_t)a - (uint32_t)((int32_t)p.zx[g] * p.rowsum[col]));
        if (p.acc) p.acc[row * p.n + col] = a;
        if (p.y) {
            const float sc = p.sx[g] * p.sw[col];
            float v = (float)a * sc;
            if (p.bias) v = v + p.bias[col];
            p.y[row * p.n + col] = v;
        }
    };

    if (sp.slices == 1) {
        if (!col_ok) return;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_of(mb, r);
                if (row < p.m) epilogue(row, acc[mb][r]);
            }
        return;
    }

    // Publish the partial tile with agent-scope stores (they go to the
    // device coherence point, so no cache writeback is needed), wait for
    // them to complete, then count this workgroup's arrival (wave 0 only).
    if (col_ok) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_of(mb, r);
                if (row < p.m)
                    __hip_atomic_store(sp.part + (slice * p.m + row) * p.n + col, acc[mb][r], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(sp.counters + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (int)sp.slices - 1;
    last = __shfl(last, 0);
    if (!last) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (col_ok) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_of(mb, r);
                if (row >= p.m) continue;
                const int32_t *src = sp.part + row * p.n + col;
                // integer sum: exact whatever the order; wrapping as int32
                uint32_t a = 0;
                for (int64_t j = 0; j < sp.slices; ++j)
                    a += (uint32_t)__hip_atomic_load(src + j * p.m * p.n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                epilogue(row, (int32_t)a);
            }
    }
    if (lane == 0) __hip_atomic_store(sp.counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K bytes per workgroup: all of K when there are at least ~512 column
// blocks, otherwise enough slices for ~512 workgroups, each at least 1024
// bytes (4 waves x 4 k-steps), a multiple of 64.
int64_t choose_kslice(int64_t nblk, int64_t k) {
    int64_t s = (512 + nblk - 1) / nblk;
    s = std::max<int64_t>(1, std::min<int64_t>(s, k / 1024));
    int64_t ks = (k + s - 1) / s;
    return (ks + 63) & ~(int64_t)63;
}

int launch(const QParams &p, hipStream_t s) {
    SkParams sp{};
    sp.q = p;
    sp.nblk = (p.n + kCols - 1) / kCols;
    sp.kslice = choose_kslice(sp.nblk, p.k);
    sp.slices = (p.k + sp.kslice - 1) / sp.kslice;
    if (sp.slices > 1) {
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(int32_t) * (size_t)(sp.slices * p.m * p.n), &ws));
        sp.part = static_cast<int32_t *>(ws);
        GFH_TRY(stream_counters(s, (size_t)sp.nblk, &sp.counters));
    }
    const dim3 grid((unsigned)(sp.nblk * sp.slices)), block(kThreads);
    if (p.m <= 16)
        hipLaunchKernelGGL(qlinear_skinny_kernel<1>, grid, block, 0, s, sp);
    else if (p.m <= 32)
        hipLaunchKernelGGL(qlinear_skinny_kernel<2>, grid, block, 0, s, sp);
    else
        hipLaunchKernelGGL(qlinear_skinny_kernel<4>, grid, block, 0, s, sp);
    return check_launch("qlinear_i8 (skinny)");
}

}  // namespace skinny

}  // namespace

int launch_qlinear_i8(const QLinearDesc &d, hipStream_t s) {
    QParams p{};
    p.qx = d.qx;
    p.sx = d.sx;
    p.zx = d.zx;
    p.qw = d.qw;
    p.sw = d.sw;
    p.rowsum = d.w_rowsum;
    p.bias = d.bias;
    p.y = d.y;
    p.acc = d.acc;
    p.m = d.m;
    p.n = d.n;
    p.k = d.k;
    p.x_per_row = d.x_per_row ? 1 : 0;
    if (d.m <= 64 && d.k % 16 == 0 && d.k > 0 && aligned16(d.qx) && aligned16(d.qw)) return skinny::launch(p, s);
    if (d.m >= 1024 && d.k % big::kBK == 0 && d.k > 0 && aligned16(d.qx) && aligned16(d.qw)) {
        p.tiles_m = (int)((d.m + big::kBM - 1) / big::kBM);
        p.tiles_n = (int)((d.n + big::kBN - 1) / big::kBN);
        const dim3 grid((unsigned)(p.tiles_m * p.tiles_n));
        if (d.x_per_row) {
            if (d.acc)
                hipLaunchKernelGGL((big::qlinear_tile256_kernel<true, true>), grid, dim3(kThreads), 0, s, p);
            else
                hipLaunchKernelGGL((big::qlinear_tile256_kernel<true, false>), grid, dim3(kThreads), 0, s, p);
        } else {
            if (d.acc)
                hipLaunchKernelGGL((big::qlinear_tile256_kernel<false, true>), grid, dim3(kThreads), 0, s, p);
            else
                hipLaunchKernelGGL((big::qlinear_tile256_kernel<false, false>), grid, dim3(kThreads), 0, s, p);
        }
        return check_launch("qlinear_i8");
    }
    p.tiles_m = (int)((d.m + kBM - 1) / kBM);
    p.tiles_n = (int)((d.n + kBN - 1) / kBN);
    const bool vec = (d.k % 16 == 0) && aligned16(d.qx) && aligned16(d.qw);
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n));
    if (vec)
        hipLaunchKernelGGL(qlinear_mfma_kernel<true>, grid, dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL(qlinear_mfma_kernel<false>, grid, dim3(kThreads), 0, s, p);
    return check_launch("qlinear_i8");
}

}  // namespace gfh
