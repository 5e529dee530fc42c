// qgemm.hip -- INT8 linear on CDNA4 i8 MFMA (v_mfma_i32_16x16x64_i8; the generic
// fallback for K % 64 != 0 on v_mfma_i32_32x32x32_i8).
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
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "quant_math.hpp"

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
    // SwiGLU gate/up mode (the `*2` operand is up_proj, the first gate_proj):
    // y = silu(gate) * up, and per-workgroup (min, max) of y into hpart.
    const int8_t *qw2;
    const float *sw2;
    const int32_t *rowsum2;
    const float *bias2;
    float2 *hpart;
    // Activations quantized inside the kernel (the 16-column skinny kernel
    // only): fp32 x [m, k], quantized per tensor, asymmetric, from the
    // (min, max) of all of x, or of the xpart partials when given.
    const float *xf;
    const float2 *xpart;
    int nxpart;
    // K split over workgroups (the tile kernel, slices > 1): slice j covers K
    // elements [j kslice, (j + 1) kslice) of every tile; each publishes its
    // int32 accumulators to part and the last to arrive on counters[tile]
    // adds them and runs the epilogue.
    int slices;
    int64_t kslice;
    int32_t *part;
    int *counters;
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


// ---- MFMA tiles fed by direct-to-LDS loads (M > 64) ------------------------------
//
// A workgroup owns a BM x BN output tile; its NWM x NWN waves each hold a
// (BM/NWM) x (BN/NWN) sub-tile as v_mfma_i32_16x16x64_i8 accumulators.
// The dispatch runs 8 waves in a 2 x 4 grid: 256 x 256 tiles (M > 512)
// give each wave 8 x 4 accumulators (128 registers), 128 x 128 tiles 4 x 2.
// The 16 x 16 x 64 form, rather than 32 x 32 x 32 (the same operations per
// wave tile, the same LDS reads), because the clock holds up better under
// it: a register-only loop of each on quantized-Gaussian operands sustained
// 4277 against 3584 TOP/s (uniform random codes 4058 / 3254; all-zero
// operands 4909 / 4924), and the int8 GEMMs at 4096 rows are power-bound.
// Operands stream through rings of SA (A) and SB (B) slots of BK bytes of K,
// filled with global_load_lds_dwordx4 (global memory straight into LDS, no
// VGPR staging); all stages but the one being consumed are in flight.  At
// 256 x 256 x 128 two full stages take 128 KB, so the remaining 32 KB of the
// 160 KB LDS holds a third A slot: A stages are requested two stages ahead,
// B stages one.  One load
// instruction fills 1 KB of LDS = 1024/BK rows of BK bytes.  BK = 128 makes
// every row run a whole 128-byte line, which measured 1.6-1.8x the ingest
// rate per CU of BK = 64 (half lines); BK = 64 serves K % 128 == 64.  Chunk
// c (16 bytes) of row r is stored at position c ^ swz(r), which spreads the
// 16-byte fragment reads over distinct banks; each lane of a load fetches
// the chunk that lands at its own LDS slot, so the swizzle costs nothing on
// the load side.  Rows past M / N are clamped to the last row (their
// products are never stored).
namespace big {

constexpr int kGroupM = 4;

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(1))) void *glb_ptr;

// Chunk swizzle of a BK-byte LDS row.  A wave's fragment read has lanes 0-31
// on rows 0-31 of a block at one logical chunk (lanes 32-63 at the next);
// gfx950's LDS serves a ds_read_b128 16 lanes at a time over 64 banks, and
// these swizzles put those 16 lanes on 16 distinct 4-bank groups (measured
// conflict-free: 4.3 clk per ds_read_b128 per CU, against 15.8 unswizzled).
template <int BK>
__device__ __forceinline__ int swz(int r) {
    return BK == 64 ? ((r >> 2) & 3) : ((r >> 1) & 7);
}

// s_waitcnt with only vmcnt constrained (expcnt / lgkmcnt left at maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Scheduling groups for one k-step: NM MFMAs, with NV global loads and ND
// LDS fragment reads spread evenly between them, so that LDS latency and
// load issue hide behind the MFMA pipe instead of stalling it.
template <int NV, int ND, int NM, int G = 0>
__device__ __forceinline__ void interleave() {
    if constexpr (G < NM) {
        constexpr int v = (G + 1) * NV / NM - G * NV / NM;
        constexpr int d = (G + 1) * ND / NM - G * ND / NM;
        if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x010, v, 0);  // VMEM
        if constexpr (d > 0) __builtin_amdgcn_sched_group_barrier(0x100, d, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // MFMA
        interleave<NV, ND, NM, G + 1>();
    }
}

// SA / SB: ring slots of the A / B operand.  With SA == SB + 1, A stages
// are requested one stage further ahead than B stages in the same LDS.
template <int BM, int BN, int BK, int SA, int SB, int NWM = 2, int NWN = 2>
struct Tile {
    static_assert(BK == 64 || BK == 128, "stage depth in K");
    static_assert(SB >= 2 && (SA == SB || SA == SB + 1), "ring slots");
    static constexpr int kNW = NWM * NWN, kNT = 64 * kNW;   // waves, threads
    static constexpr int kWM = BM / NWM, kWN = BN / NWN;     // wave sub-tile
    static constexpr int kFM = kWM / 16, kFN = kWN / 16;     // 16 x 16 accumulators per wave
    static constexpr int kSteps = BK / 64;                   // MFMA k-steps per stage
    static constexpr int kChunks = BK / 16;                  // 16-byte chunks per row
    static constexpr int kRowsPerLoad = 1024 / BK;           // rows filled by one load instruction
    static constexpr int kLA = BM * BK / (1024 * kNW), kLB = BN * BK / (1024 * kNW);  // loads per wave per stage
    static constexpr int kLPS = kLA + kLB;
    static constexpr int kABytes = BM * BK, kBBytes = BN * BK;
    static constexpr int kRing = SA * kABytes + SB * kBBytes;
    // Loads of this wave still allowed in flight when stage t+1 must have
    // landed (end of stage t).  Stage s's B part is requested at the end of
    // stage s - SB, its A part at the end of stage s - SA, each batch B
    // first; in-order completion makes the count exact.
    static constexpr int kWaitSteady = (SA - SB) * kLA + (SB - 2) * (kLA + kLB);
    // The same before the first stage, after the prologue's requests.
    static constexpr int kWaitFirst = (SB - 1) * (kLA + kLB) + (SA - SB) * kLA;
    // Output staging: each wave converts half of its sub-tile (kWM/2 rows x
    // kWN columns) at a time -- all of it when it is a single 16-row block;
    // a row stride of kWN + 4 floats (4 rows apart: 16 banks apart) keeps
    // the four row groups of one ds_write_b32 on disjoint banks.
    static constexpr int kOutPasses = kFM >= 2 ? 2 : 1;
    static constexpr int kOutRows = kWM / kOutPasses;
    static constexpr int kOutStride = kWN + 4;
    static constexpr int kOut = kNW * kOutRows * kOutStride * 4;
    static constexpr int kLds = kRing > kOut ? kRing : kOut;
    static_assert(kLds <= 160 * 1024, "LDS per workgroup");
};

// DUAL (SwiGLU gate/up): the B tile's 32-row blocks alternate between
// gate_proj and up_proj rows of the same BN / 2 output columns, so a wave's
// accumulator blocks j = 0, 1 hold gate and j = 2, 3 up of one 32-column
// group (16 columns each) and the epilogue writes silu(gate) * up straight
// from registers.
template <int BM, int BN, int BK, int SA, int SB, int NWM, int NWN, bool X_PER_ROW, bool WANT_ACC, bool DUAL = false>
__global__ __launch_bounds__((Tile<BM, BN, BK, SA, SB, NWM, NWN>::kNT),
                             ((Tile<BM, BN, BK, SA, SB, NWM, NWN>::kLds > 80 * 1024) ? 1 : 2)) void qlinear_tile_kernel(
    QParams p) {
    using T = Tile<BM, BN, BK, SA, SB, NWM, NWN>;
    static_assert(!DUAL || (!X_PER_ROW && !WANT_ACC && NWN * 64 == BN), "dual mode: wave = 2 column blocks");
    constexpr int NW = T::kNW;
    constexpr int FM = T::kFM, FN = T::kFN, WM = T::kWM, WN = T::kWN;
    constexpr int RPL = T::kRowsPerLoad, CPR = T::kChunks;
    __shared__ __attribute__((aligned(1024))) int8_t lds[T::kLds];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = (wave / NWN) * WM;
    const int wn0 = (wave % NWN) * WN;

    const int nblk = p.tiles_m * p.tiles_n;
    // Workgroup -> (slice, tile): each XCD takes a contiguous range of
    // slice-major ids, so tiles of one slice that share rows of x or W run
    // under one L2.
    const int vid = xcd_chunked(blockIdx.x, nblk * p.slices);
    const int slice = vid / nblk;
    const int bid = vid - slice * nblk;
    const int group_size = kGroupM * p.tiles_n;
    const int group = bid / group_size;
    const int first_m = group * kGroupM;
    const int gm = min(p.tiles_m - first_m, kGroupM);
    const int in_group = bid - group * group_size;
    const int64_t m0 = (int64_t)(first_m + in_group % gm) * BM;
    // first output column (in dual mode BN / 2 columns of gate and of up)
    const int64_t n0 = (int64_t)(in_group / gm) * (DUAL ? BN / 2 : BN);

    // Byte offsets, relative to the tile's first row, of this wave's load
    // instructions: A instruction j covers tile rows wave*(BM/NW) + j*RPL ..
    // +RPL-1; lane l fills LDS slot l of that 1 KB run (row l / CPR, physical
    // chunk l % CPR) from logical chunk (l % CPR) ^ swz(row).  The host
    // guarantees BM * K < 2^32.
    const int64_t k_lo = (int64_t)slice * p.kslice;  // a multiple of BK
    const int8_t *a_base = p.qx + m0 * p.k + k_lo;
    const int8_t *b_src[T::kLB];  // per load instruction: its matrix at row n0 (uniform)
    uint32_t a_off[T::kLA], b_off[T::kLB];
#pragma unroll
    for (int j = 0; j < T::kLA; ++j) {
        const int r = wave * (BM / NW) + j * RPL + lane / CPR;
        a_off[j] = (uint32_t)((min(m0 + r, p.m - 1) - m0) * p.k) + (uint32_t)(((lane % CPR) ^ swz<BK>(r)) * 16);
    }
#pragma unroll
    for (int j = 0; j < T::kLB; ++j) {
        const int r0 = wave * (BN / NW) + j * RPL;  // multiple of RPL: one 32-row block per instruction
        const int r = r0 + lane / CPR;
        const int rl = DUAL ? ((r >> 6) << 5) + (r & 31) : r;  // row of its matrix, from n0
        b_src[j] = (DUAL && ((r0 >> 5) & 1) ? p.qw2 : p.qw) + n0 * p.k + k_lo;
        b_off[j] = (uint32_t)((min(n0 + rl, p.n - 1) - n0) * p.k) + (uint32_t)(((lane % CPR) ^ swz<BK>(r)) * 16);
    }
    const int nk = (int)(min(p.kslice, p.k - k_lo) / BK);

    // Ring slots: A stages at [0, SA * kABytes), B stages after them.
    int8_t *const ring_b = lds + SA * T::kABytes;
    // Request K stage t of A (of B) into ring slot `slot`.
    auto issue_a = [&](int t, int slot) {
        int8_t *la = lds + slot * T::kABytes;
        const int8_t *ga = a_base + (int64_t)t * BK;
#pragma unroll
        for (int j = 0; j < T::kLA; ++j)
            __builtin_amdgcn_global_load_lds((glb_ptr)(ga + a_off[j]), (lds_ptr)(la + (wave * (BM / NW) + j * RPL) * BK),
                                             16, 0, 0);
    };
    auto issue_b = [&](int t, int slot) {
        int8_t *lb = ring_b + slot * T::kBBytes;
#pragma unroll
        for (int j = 0; j < T::kLB; ++j)
            __builtin_amdgcn_global_load_lds((glb_ptr)(b_src[j] + (int64_t)t * BK + b_off[j]),
                                             (lds_ptr)(lb + (wave * (BN / NW) + j * RPL) * BK), 16, 0, 0);
    };

    // Fragment address inside a stage: lane l reads row l%16 of a 16-row
    // block, logical chunk 4*ks + l/16 (the operand layout of
    // v_mfma_i32_16x16x64_i8: 16 consecutive k bytes per lane).  Blocks
    // start at multiples of 16 rows, so the swizzle depends on l only; the
    // 16 lanes of one chunk then read 16 rows on 16 distinct 4-bank groups
    // (BK = 128: even rows on banks 4 (c ^ s), odd rows 32 above; BK = 64:
    // row 4a + b on 16 b + 4 (c ^ a)).
    const int frow = lane & 15, fq = lane >> 4, fsw = swz<BK>(frow);
    auto frag_off = [&](int ks) { return frow * BK + (((((ks << 2) | fq)) ^ fsw) << 4); };

    i32x4 af[2][FM], bf[2][FN];
    auto load_frags = [&](int buf, int t, int ks) {
        const int8_t *la = lds + (t % SA) * T::kABytes;
        const int8_t *lb = ring_b + (t % SB) * T::kBBytes;
        const int fo = frag_off(ks);
#pragma unroll
        for (int i = 0; i < FM; ++i) af[buf][i] = *reinterpret_cast<const i32x4 *>(la + (wm0 + i * 16) * BK + fo);
#pragma unroll
        for (int j = 0; j < FN; ++j) bf[buf][j] = *reinterpret_cast<const i32x4 *>(lb + (wn0 + j * 16) * BK + fo);
    };

    i32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    auto mfmas = [&](int buf) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[buf][i], bf[buf][j], acc[i][j], 0, 0, 0);
    };

    // Stages t+SB of B and t+SA of A are issued into stage t's slots as soon
    // as every wave holds the last fragments of stage t.  Within a stage,
    // the fragments of k-step ks+1 are read while the MFMAs of k-step ks
    // run.  The loop body has no branches so that the scheduler can
    // interleave reads, loads and MFMAs across it: past the end of K the
    // ring reloads the last stage into the slot just freed (never read
    // again), which keeps the number of loads in flight, and so every wait
    // count, constant.
    for (int t = 0; t < SB; ++t) {
        issue_a(min(t, nk - 1), t);
        issue_b(min(t, nk - 1), t);
    }
    for (int t = SB; t < SA; ++t) issue_a(min(t, nk - 1), t);
    wait_vmcnt<T::kWaitFirst>();
    __builtin_amdgcn_s_barrier();
    load_frags(0, 0, 0);

    constexpr int NR = FM + FN, NM = FM * FN;
    auto k_steps = [&](int t) {
#pragma unroll
        for (int ks = 0; ks + 1 < T::kSteps; ++ks) {
            load_frags((ks + 1) & 1, t, ks + 1);
            mfmas(ks & 1);
            interleave<0, NR, NM>();
        }
    };
    for (int t = 0; t + 1 < nk; ++t) {
        k_steps(t);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();  // this wave's reads of stage t are done
        // stage t+1 landed; later requests may still be in flight
        wait_vmcnt<T::kWaitSteady>();
        __builtin_amdgcn_s_barrier();
        issue_b(min(t + SB, nk - 1), t % SB);
        issue_a(min(t + SA, nk - 1), t % SA);
        if constexpr (T::kSteps >= 2) {
            load_frags(0, t + 1, 0);
            mfmas((T::kSteps - 1) & 1);
        } else {  // one k-step per stage (BK = 64): this stage's MFMAs, then the next stage's fragments
            mfmas(0);
            load_frags(0, t + 1, 0);
        }
        interleave<T::kLPS, NR, NM>();
        __builtin_amdgcn_sched_barrier(0);
    }
    k_steps(nk - 1);
    mfmas((T::kSteps - 1) & 1);
    // No load may still be writing the ring when the workgroup moves on.
    wait_vmcnt<0>();

    if constexpr (!DUAL) {
        if (p.slices > 1) {
            // Split K: publish this slice's int32 accumulators (register r of
            // thread t at [slot][r][t], 2 KB per register and workgroup, so
            // the stores and loads are coalesced), count the arrival, and
            // let the last slice of the tile add the others' (integer, so
            // exact in any order) and run the epilogue.  The arrival
            // protocol is common.hpp's.
            constexpr int REGS = FM * FN * 4, R4 = FM * FN;
            constexpr int NT = T::kNT;
            // 16-byte stores and loads at the coherence point (common.hpp):
            // accumulator block q = i FN + j of thread t at [slot][q][t].
            const __amdgpu_buffer_rsrc_t part_buf =
                coherent_buffer(p.part, (uint32_t)((int64_t)p.slices * nblk * REGS * NT * 4));
            auto part_off = [&](int64_t sl, int q4) {
                return (uint32_t)((((sl * nblk + bid) * R4 + q4) * NT + tid) * 16);
            };
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    __builtin_amdgcn_raw_buffer_store_b128(acc[i][j], part_buf, part_off(slice, i * FN + j), 0,
                                                           kScDevice);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            wait_vmcnt<0>();  // this thread's partial stores are complete
            // (the flag goes through the operand ring: after this barrier no
            // wave reads a fragment from it any more)
            int *last_flag = reinterpret_cast<int *>(lds);
            __syncthreads();
            if (tid == 0)
                *last_flag = __hip_atomic_fetch_add(p.counters + bid, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                             p.slices - 1;
            __syncthreads();
            if (!*last_flag) return;
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            // The other slices' partials, G slices at a time with every load
            // of a group requested before the first add.
            constexpr int G = REGS >= 96 ? 1 : 96 / REGS;
            for (int j0 = 0; j0 < p.slices; j0 += G) {
                i32x4 t[G][R4];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const int j = j0 + g;
                    const bool use = j < p.slices && j != slice;
#pragma unroll
                    for (int q4 = 0; q4 < R4; ++q4)
                        t[g][q4] = use ? __builtin_amdgcn_raw_buffer_load_b128(part_buf, part_off(j, q4), 0, kScDevice)
                                       : i32x4{0, 0, 0, 0};
                }
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int jj = 0; jj < FN; ++jj) {
                            const i32x4 w = t[g][i * FN + jj];
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const int32_t e = w[r];
                                acc[i][jj][r] = (int32_t)((uint32_t)acc[i][jj][r] + (uint32_t)e);
                            }
                        }
            }
            if (tid == 0) __hip_atomic_store(p.counters + bid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    if constexpr (DUAL) {
        // Lane l, register r of block (i, j): row 4*(l/16) + r, column l%16
        // of the 16 x 16 block; blocks j < FN/2 are gate, j + FN/2 the up
        // projection of the same columns.
        constexpr int FG = FN / 2;
        const int32_t zx0 = p.zx ? (int32_t)p.zx[0] : 0;
        const float sx0 = p.sx[0];
        int64_t col[FG];
        int32_t rs_g[FG], rs_u[FG];
        float sc_g[FG], sc_u[FG], b_g[FG], b_u[FG];
#pragma unroll
        for (int j = 0; j < FG; ++j) {
            col[j] = n0 + wn0 / 2 + j * 16 + (lane & 15);
            const int64_t cc = min(col[j], p.n - 1);
            rs_g[j] = p.zx ? p.rowsum[cc] : 0;
            rs_u[j] = p.zx ? p.rowsum2[cc] : 0;
            sc_g[j] = sx0 * p.sw[cc];
            sc_u[j] = sx0 * p.sw2[cc];
            b_g[j] = p.bias ? p.bias[cc] : 0.f;
            b_u[j] = p.bias2 ? p.bias2[cc] : 0.f;
        }
        float mn = INFINITY, mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FG; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + wm0 + i * 16 + 4 * (lane >> 4) + r;
                    const int32_t ag = (int32_t)((uint32_t)acc[i][j][r] - (uint32_t)(zx0 * rs_g[j]));
                    const int32_t au = (int32_t)((uint32_t)acc[i][j + FG][r] - (uint32_t)(zx0 * rs_u[j]));
                    float g = (float)ag * sc_g[j];
                    float u = (float)au * sc_u[j];
                    if (p.bias) g = g + b_g[j];
                    if (p.bias2) u = u + b_u[j];
                    const float h = silu_mul1(g, u);
                    if (row < p.m && col[j] < p.n) {
                        p.y[row * p.n + col[j]] = h;
                        mn = fminf(mn, h);
                        mx = fmaxf(mx, h);
                    }
                }
        wave_minmax(mn, mx);
        // Cross-wave fold through the (now idle) operand ring.
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        float2 *red = reinterpret_cast<float2 *>(lds);
        if (lane == 0) red[wave] = make_float2(mn, mx);
        __syncthreads();
        if (tid == 0) {
            float2 t = red[0];
#pragma unroll
            for (int w = 1; w < NW; ++w) t = make_float2(fminf(t.x, red[w].x), fmaxf(t.y, red[w].y));
            p.hpart[blockIdx.x] = t;
        }
        return;
    }

    // Epilogue: lane l, register r of block (i, j) holds
    // row 4*(l/16) + r, column l%16 of that 16 x 16 block.
    // Per-tensor activation parameters are uniform; per-row ones are read
    // once per row.
    const int zx0 = (!X_PER_ROW && p.zx) ? (int)p.zx[0] : 0;
    const float sx0 = (!X_PER_ROW && p.y) ? p.sx[0] : 0.f;
    int32_t rs[FN];
    float swc[FN], bc[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t col = min(n0 + wn0 + j * 16 + (lane & 15), p.n - 1);
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
            const int64_t row = min(m0 + wm0 + i * 16 + 4 * (lane >> 4) + r, p.m - 1);
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
        for (int j = 0; j < FN; ++j) {
            const int64_t col = n0 + wn0 + j * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + wm0 + i * 16 + 4 * (lane >> 4) + r;
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

    // Output tile through LDS: each wave converts half of its sub-tile (all
    // of a single 16-row block) at a time into its own region, then writes
    // whole row runs (WN floats) with 16-byte stores.
    constexpr int LPR = WN / 4;                // lanes per output row
    constexpr int RPI = 64 / LPR;              // rows per read instruction
    constexpr int PASSES = T::kOutPasses;
    constexpr int HALF = T::kOutRows;          // rows per pass
    constexpr int BPP = FM / PASSES;           // 16-row blocks per pass
    static_assert(BPP * PASSES == FM && BPP * 16 == HALF, "output passes cover the sub-tile");
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();  // every wave is done with the operand ring
    float *lt = reinterpret_cast<float *>(lds) + wave * (HALF * T::kOutStride);
    const bool vec_out = (p.n % 4) == 0;
#pragma unroll
    for (int h = 0; h < PASSES; ++h) {
#pragma unroll
        for (int ii = 0; ii < BPP; ++ii)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int32_t a;
                    const float v = finish(h * BPP + ii, j, r, a);
                    const int lr = ii * 16 + 4 * (lane >> 4) + r;
                    lt[lr * T::kOutStride + j * 16 + (lane & 15)] = v;
                }
        const int64_t col = n0 + wn0 + 4 * (lane % LPR);
#pragma unroll
        for (int q = 0; q < HALF / RPI; ++q) {
            const int lr = RPI * q + lane / LPR;
            const f32x4 v = *reinterpret_cast<const f32x4 *>(lt + lr * T::kOutStride + 4 * (lane % LPR));
            const int64_t row = m0 + wm0 + h * HALF + lr;
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

// slices > 1: K split into that many slices of whole BK stages (the caller
// keeps tiles x slices within one round of workgroups).
template <int BM, int BN, int BK, int SA, int SB, int NWM = 2, int NWN = 2>
int launch_tiles(QParams p, hipStream_t s, int slices = 1) {
    using T = Tile<BM, BN, BK, SA, SB, NWM, NWN>;
    p.tiles_m = (int)((p.m + BM - 1) / BM);
    p.tiles_n = (int)((p.n + BN - 1) / BN);
    const int64_t stages = p.k / BK;
    if (slices > stages) slices = (int)stages;
    p.kslice = slices > 1 ? (stages + slices - 1) / slices * BK : p.k;
    p.slices = slices > 1 ? (int)((p.k + p.kslice - 1) / p.kslice) : 1;
    p.part = nullptr;
    p.counters = nullptr;
    const int64_t nblk = (int64_t)p.tiles_m * p.tiles_n;
    if (p.slices > 1) {
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(int32_t) * (size_t)(p.slices * nblk) * BM * BN, &ws));
        p.part = static_cast<int32_t *>(ws);
        GFH_TRY(stream_counters(s, (size_t)nblk, &p.counters));
    }
    const dim3 grid((unsigned)(nblk * p.slices)), block(T::kNT);
    if (p.x_per_row) {
        if (p.acc)
            hipLaunchKernelGGL((qlinear_tile_kernel<BM, BN, BK, SA, SB, NWM, NWN, true, true>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((qlinear_tile_kernel<BM, BN, BK, SA, SB, NWM, NWN, true, false>), grid, block, 0, s, p);
    } else {
        if (p.acc)
            hipLaunchKernelGGL((qlinear_tile_kernel<BM, BN, BK, SA, SB, NWM, NWN, false, true>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((qlinear_tile_kernel<BM, BN, BK, SA, SB, NWM, NWN, false, false>), grid, block, 0, s, p);
    }
    return check_launch("qlinear_i8");
}

// Dual (SwiGLU gate/up) launch: p.n logical columns of each matrix, BN / 2
// per tile; one hpart entry per workgroup.
template <int BM, int BN, int BK, int SA, int SB, int NWM, int NWN>
int launch_tiles_dual(QParams p, hipStream_t s, int *npart) {
    p.tiles_m = (int)((p.m + BM - 1) / BM);
    p.tiles_n = (int)((p.n + BN / 2 - 1) / (BN / 2));
    p.slices = 1;
    p.kslice = p.k;
    *npart = p.tiles_m * p.tiles_n;
    const dim3 grid((unsigned)(p.tiles_m * p.tiles_n)), block(Tile<BM, BN, BK, SA, SB, NWM, NWN>::kNT);
    hipLaunchKernelGGL((qlinear_tile_kernel<BM, BN, BK, SA, SB, NWM, NWN, false, false, true>), grid, block, 0, s, p);
    return check_launch("qlinear_swiglu_i8");
}

}  // namespace big


// ---- skinny M (decode): weights streamed from HBM straight into MFMA ----------
//
// For M <= 64 the layer is HBM-bound (the weight is read once, 45 MB for
// W [11008, 4096]).  W [N, K] is K-contiguous, which is exactly the per-lane
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

struct SkParams {
    QParams q;
    int64_t kslice, slices, nblk;
    int32_t *part;  // [slices][D][m][n] partial accumulators (slices > 1)
    int *counters;  // one per column block, zero at rest (slices > 1)
};

// DUAL (SwiGLU gate/up): each wave multiplies the same x fragments with the
// gate rows and the up rows of its 16 columns (D = 2 accumulator sets), and
// the epilogue writes silu(gate) * up plus the workgroup's (min, max) of it.
// QX: the activations arrive in fp32 (p.xf) and are quantized per tensor
// (asymmetric, quantize_activation, quantization.rs:280-287) by every
// workgroup itself: the (min, max) of all of x (or the fold of p.xpart),
// the scale and zero point, and the codes of this workgroup's K-slice into
// LDS, with the quantize kernels' own arithmetic (quant_math.hpp), so the
// codes are those of gfh_quantize_i8_per_tensor.  It replaces the two
// quantize launches ahead of the INT8 linear at decode sizes.
constexpr int kQxBytes = 32768;  // LDS for the codes: m x kslice bytes
// (QX: four workgroups per CU, as without it -- at 136 registers three fit,
// and N = 14336's 896 workgroups then needed a second round.)
template <int MB, bool DUAL, bool QX = false>
__global__ __launch_bounds__(kThreads, QX ? 4 : 1) void qlinear_skinny_kernel(SkParams sp) {
    static_assert(!QX || MB == 1, "in-kernel quantization: at most 16 rows of x");
    constexpr int D = DUAL ? 2 : 1;
    // k-steps in flight per lane (QX with two weights: 4, so that four
    // workgroups fit per CU without spilling)
    constexpr int kU = (DUAL && (MB > 2 || QX)) ? 4 : 8;
    const QParams &p = sp.q;
    __shared__ i32x4 red[kWaves - 1][D * MB][64];
    __shared__ __attribute__((aligned(16))) int8_t xq[QX ? kQxBytes : 16];
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
    const int64_t wrow = min(n0 + (lane & 15), p.n - 1) * p.k + k_lo + kb;
    const int8_t *wsrc[D];
    wsrc[0] = p.qw + wrow;
    if (DUAL) wsrc[D - 1] = p.qw2 + wrow;
    const int8_t *xsrc = p.qx + k_lo + kb;

    float qx_scale = 0.f;
    int32_t qx_zp = 0;
    if constexpr (QX) {
        float mn = INFINITY, mx = -INFINITY;
        if (p.xpart) {
            for (int i = threadIdx.x; i < p.nxpart; i += kThreads) {
                const float2 v = p.xpart[i];
                mn = fminf(mn, v.x);
                mx = fmaxf(mx, v.y);
            }
        } else {
            // x is [m, k] contiguous with k % 16 == 0 and 16-byte aligned.
            const f32x4 *xv = reinterpret_cast<const f32x4 *>(p.xf);
            const int64_t nv = p.m * p.k / 4;
            for (int64_t i = threadIdx.x; i < nv; i += kThreads) {
                const f32x4 v = xv[i];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float ve = v[e];
                    mn = fminf(mn, ve);
                    mx = fmaxf(mx, ve);
                }
            }
        }
        qmath::block_minmax<kThreads>(mn, mx);
        int8_t zp8;
        qmath::quant_params(mn, mx, false, qx_scale, zp8);
        qx_zp = zp8;
        // Codes of rows [0, m) x [k_lo, k_lo + kl), row r at xq + r * kslice.
        const int q4 = kl / 4;
        for (int i = threadIdx.x; i < (int)p.m * q4; i += kThreads) {
            const int r = i / q4, c = 4 * (i - r * q4);
            const f32x4 v = *reinterpret_cast<const f32x4 *>(p.xf + r * p.k + k_lo + c);
            *reinterpret_cast<uint32_t *>(xq + r * sp.kslice + c) = qmath::quant4(v, qx_scale, qx_zp);
        }
        __syncthreads();
    }

    i32x4 acc[D][MB];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[d][mb] = i32x4{0, 0, 0, 0};
    for (int s0 = st0; s0 < st1; s0 += kU) {
        i32x4 w[kU][D], xf[kU][MB];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int off = (s0 + u) * 64;
            const bool ok = s0 + u < st1 && off + kb < kl;
#pragma unroll
            for (int d = 0; d < D; ++d)
                w[u][d] = ok ? __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wsrc[d] + off)) : i32x4{0, 0, 0, 0};
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int64_t row = mb * 16 + (lane & 15);
                if constexpr (QX)
                    xf[u][mb] = (ok && row < p.m) ? *reinterpret_cast<const i32x4 *>(xq + row * sp.kslice + off + kb)
                                                  : i32x4{0, 0, 0, 0};
                else
                    xf[u][mb] = (ok && row < p.m) ? *reinterpret_cast<const i32x4 *>(xsrc + row * p.k + off)
                                                  : i32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int d = 0; d < D; ++d)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[d][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xf[u][mb], w[u][d], acc[d][mb], 0, 0, 0);
    }

    // Add the four waves' accumulators (exact int32) in wave 0.
    if (wave > 0) {
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) red[wave - 1][d * MB + mb][lane] = acc[d][mb];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int w2 = 0; w2 < kWaves - 1; ++w2) acc[d][mb] += red[w2][d * MB + mb][lane];

    // 16x16 accumulator layout: lane l, register r -> row 4 * (l / 16) + r,
    // column l % 16 of the block.
    const int64_t col = n0 + (lane & 15);
    const bool col_ok = col < p.n;
    auto row_of = [&](int mb, int r) -> int64_t { return (int64_t)mb * 16 + 4 * (lane >> 4) + r; };
    // Zero-point-corrected accumulator of matrix d (0 = qw, 1 = qw2), and its
    // dequantized value plus bias.
    auto corrected = [&](int d, int64_t row, int32_t raw) -> int32_t {
        if (!QX && !p.zx) return raw;
        const int32_t *rs = d ? p.rowsum2 : p.rowsum;
        const int32_t zx = QX ? qx_zp : (int32_t)p.zx[p.x_per_row ? row : 0];
        return (int32_t)((uint32_t)raw - (uint32_t)(zx * rs[col]));
    };
    auto dequant = [&](int d, int64_t row, int32_t a) -> float {
        const float *sw = d ? p.sw2 : p.sw;
        const float *bias = d ? p.bias2 : p.bias;
        const float sc = (QX ? qx_scale : p.sx[p.x_per_row ? row : 0]) * sw[col];
        float v = (float)a * sc;
        if (bias) v = v + bias[col];
        return v;
    };
    float mn = INFINITY, mx = -INFINITY;
    auto epilogue = [&](int64_t row, const int32_t *raw) {
        if (DUAL) {
            const float g = dequant(0, row, corrected(0, row, raw[0]));
            const float u = dequant(1, row, corrected(1, row, raw[D - 1]));
            const float h = silu_mul1(g, u);
            p.y[row * p.n + col] = h;
            mn = fminf(mn, h);
            mx = fmaxf(mx, h);
            return;
        }
        const int32_t a = corrected(0, row, raw[0]);
        if (p.acc) p.acc[row * p.n + col] = a;
        if (p.y) p.y[row * p.n + col] = dequant(0, row, a);
    };
    auto publish_minmax = [&]() {
        if (!DUAL) return;
        wave_minmax(mn, mx);
        if (lane == 0) p.hpart[blk] = make_float2(mn, mx);
    };

    if (sp.slices == 1) {
        if (col_ok) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = row_of(mb, r);
                    int32_t raw[D];
#pragma unroll
                    for (int d = 0; d < D; ++d) raw[d] = acc[d][mb][r];
                    if (row < p.m) epilogue(row, raw);
                }
        }
        publish_minmax();
        return;
    }

    // Publish the partial tile with agent-scope stores (they go to the
    // device coherence point, so no cache writeback is needed), wait for
    // them to complete, then count this workgroup's arrival (wave 0 only).
    if (col_ok) {
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = row_of(mb, r);
                    if (row < p.m)
                        __hip_atomic_store(sp.part + ((slice * D + d) * p.m + row) * p.n + col, acc[d][mb][r],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
    }
    // split-K arrival protocol (common.hpp): steps 2-4
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
                int32_t raw[D];
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    const int32_t *src = sp.part + (d * p.m + row) * p.n + col;
                    // integer sum: exact whatever the order; wrapping as int32
                    uint32_t a = 0;
                    for (int64_t j = 0; j < sp.slices; ++j)
                        a += (uint32_t)__hip_atomic_load(src + j * D * p.m * p.n, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                    raw[d] = (int32_t)a;
                }
                epilogue(row, raw);
            }
    }
    publish_minmax();
    if (lane == 0) __hip_atomic_store(sp.counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K bytes per workgroup: all of K when there are at least ~512 column
// blocks, or at least 256 with K <= 4096; otherwise enough slices for ~512
// workgroups, each at least 1024 bytes (4 waves x 4 k-steps), a multiple
// of 64.  N = 4096, K = 4096 (256 blocks), no split / 2 slices: M = 1 6.3 /
// 7.9 us, M = 4 7.3 / 10.7 us.  At K = 11008 and 14336 two slices stay
// ahead at M = 1 (13.8 / 14.5 and 15.3 / 16.6 us) and in the SwiGLU, whose
// down projection quantizes its slice of h in each workgroup.
int64_t choose_kslice(int64_t nblk, int64_t k) {
    if (nblk >= 256 && k <= 4096) return (k + 63) & ~(int64_t)63;
    int64_t s = (512 + nblk - 1) / nblk;
    s = std::max<int64_t>(1, std::min<int64_t>(s, k / 1024));
    int64_t ks = (k + s - 1) / s;
    return (ks + 63) & ~(int64_t)63;
}

// Whether the in-kernel quantization of x pays: every workgroup computes
// the codes of its K-slice itself (m * kslice correctly rounded divisions),
// and without producer partials also reads all of x for the min / max.
// Measured against the quantize launches + INT8 linear (us, fused /
// separate): N = 11008, K = 4096: m = 1 14.8 / 18.5, m = 2 19.4 / 18.9, m = 4
// 27.4 / 19.8; N = 4096, K = 4096: m = 2 13.1 / 15.0, m = 3 16.2 / 15.9;
// N = 4096, K = 11008, m = 1 19.9 / 20.3.  With partials (the SwiGLU down
// projection, kslice 5504 / 7168 at m = 1) it paid too.
constexpr int64_t kQxCodes = 4096, kQxCodesPartials = 8192;
bool qx_fits(int64_t m, int64_t n, int64_t k, bool partials) {
    if (m < 1 || m > 4 || k <= 0 || k % 16 != 0 || n <= 0) return false;
    const int64_t codes = m * choose_kslice((n + kCols - 1) / kCols, k);
    return codes <= (partials ? kQxCodesPartials : kQxCodes) && codes <= kQxBytes;
}

template <bool DUAL>
int launch(const QParams &p, hipStream_t s, int *npart = nullptr) {
    constexpr int D = DUAL ? 2 : 1;
    SkParams sp{};
    sp.q = p;
    sp.nblk = (p.n + kCols - 1) / kCols;
    sp.kslice = choose_kslice(sp.nblk, p.k);
    sp.slices = (p.k + sp.kslice - 1) / sp.kslice;
    if (p.xf && (!qx_fits(p.m, p.n, p.k, p.xpart != nullptr) || !aligned16(p.xf) || p.zx || p.x_per_row))
        return set_error(GFH_INVALID_DATA, "qlinear_i8: in-kernel activation quantization does not serve m=%lld "
                         "k=%lld", (long long)p.m, (long long)p.k);
    if (npart) *npart = (int)sp.nblk;
    if (sp.slices > 1) {
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(int32_t) * (size_t)(sp.slices * D * p.m * p.n), &ws));
        sp.part = static_cast<int32_t *>(ws);
        GFH_TRY(stream_counters(s, (size_t)sp.nblk, &sp.counters));
    }
    const dim3 grid((unsigned)(sp.nblk * sp.slices)), block(kThreads);
    if (p.xf)
        hipLaunchKernelGGL((qlinear_skinny_kernel<1, DUAL, true>), grid, block, 0, s, sp);
    else if (p.m <= 16)
        hipLaunchKernelGGL((qlinear_skinny_kernel<1, DUAL>), grid, block, 0, s, sp);
    else if (p.m <= 32)
        hipLaunchKernelGGL((qlinear_skinny_kernel<2, DUAL>), grid, block, 0, s, sp);
    else
        hipLaunchKernelGGL((qlinear_skinny_kernel<4, DUAL>), grid, block, 0, s, sp);
    return check_launch(DUAL ? "qlinear_swiglu_i8 (skinny)" : "qlinear_i8 (skinny)");
}

}  // namespace skinny

// ---- skinny M, x shared through LDS (5 <= M <= 64) ------------------------------
//
// From 5 rows on, reading x per wave straight from L2 (as qlinear_skinny_kernel
// does) moves m / 16 times the weight bytes again.  Here a workgroup owns 64
// output columns -- wave w the 16 columns n0 + 16 w .. + 15, all m rows of x,
// over the workgroup's K-slice, so no sums cross waves -- and the slice's x
// goes through a 3-stage LDS ring shared by the four waves:
//  * K advances in 256-byte chunks.  Lane l holds 16 bytes of weight row
//    l % 16 at byte 64 s + 16 (l / 16) of step s of the chunk and the same
//    bytes of x row l % 16 (+ 16 per row block): the operand layout of
//    v_mfma_i32_16x16x64_i8;
//  * x: global_load_lds_dwordx4 fills 4 rows x 256 bytes per instruction,
//    16-byte slots swizzled by row (conflict-free fragment reads); the
//    weight chunks (both matrices in DUAL mode) go through a ring of their
//    own the same way, each wave filling its 16 rows, two chunks ahead of
//    the MFMAs.  Loaded straight into the fragment registers, one
//    instruction covered 16 rows x 64 bytes (half lines): N = 11008, K =
//    4096, M = 16 / 32 / 64 took 14.6 / 16.5 / 20.9 us against 12.5 / 14.3
//    / 18.3 us with the ring (same box);
//  * with fewer than ~512 workgroups K is also split over workgroups; each
//    wave publishes its exact int32 partials, counts its arrival on its
//    16-column block, and the last one adds the slices (exact in any order)
//    and runs the dequantizing epilogue.
// The layout, ring and wait accounting are those of the fp32 skinny NT GEMM
// (gemm_nt_skinny.hip) on int8 operands.
namespace skinny_lds {

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(1))) void *glb_ptr;

constexpr int kWaves = 4;
constexpr int kGroupCols = 16 * kWaves;  // output columns per workgroup
constexpr int kChunk = 256;              // k bytes per chunk
constexpr int kStages = 3;               // x and weight rings (two chunks in flight)

struct Params {
    QParams q;
    int64_t ngrp, kslice, slices;
    int32_t *part;  // [slices][D][m][n] partial accumulators (slices > 1)
    int *counters;  // one per 16-column block, zero at rest (slices > 1)
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

template <int MB, bool DUAL>
__global__ __launch_bounds__(64 * kWaves, (MB <= 2 && !DUAL) ? 2 : 1) void qlinear_skinny_lds_kernel(Params sp) {
    constexpr int D = DUAL ? 2 : 1;
    constexpr int kStageBytes = 16 * MB * kChunk;
    constexpr int kWStageBytes = D * kGroupCols * kChunk;  // [D][wave][16 rows][kChunk]
    constexpr int kOps = MB + 4 * D;  // vector memory instructions per chunk and wave
    __shared__ __attribute__((aligned(1024))) int8_t xs[kStages * (kStageBytes + kWStageBytes)];
    int8_t *const wsm = xs + kStages * kStageBytes;  // the weight ring
    const QParams &p = sp.q;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t grp = blockIdx.x % sp.ngrp, slice = blockIdx.x / sp.ngrp;
    const int64_t n0 = grp * kGroupCols + 16 * wave;
    const int64_t k_lo = slice * sp.kslice;
    const int kl = (int)min(sp.kslice, p.k - k_lo);  // > 0, a multiple of 16
    const int nch = (kl + kChunk - 1) / kChunk;

    // x: instruction j of wave w fills stage rows 4 (w MB + j) .. + 3; lane l
    // fills slot l % 16 of row l / 16 of them from logical 16-byte chunk
    // (l % 16) ^ (row % 16).  Rows past m read row m - 1 (never stored);
    // bytes past the slice read its last 16 (masked in the tail).
    const int8_t *xsrc[MB];
    int xcol[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        const int r = 4 * (wave * MB + j) + (lane >> 4);
        xsrc[j] = p.qx + min<int64_t>(r, p.m - 1) * p.k + k_lo;
        xcol[j] = 16 * ((lane & 15) ^ (r & 15));
    }
    auto issue_x = [&](int i, int slot) __attribute__((always_inline)) {
        int8_t *stage = xs + slot * kStageBytes;
#pragma unroll
        for (int j = 0; j < MB; ++j)
            __builtin_amdgcn_global_load_lds((glb_ptr)(xsrc[j] + min(i * kChunk + xcol[j], kl - 16)),
                                             (lds_ptr)(stage + 4 * (wave * MB + j) * kChunk), 16, 0, 0);
    };
    // W goes through an LDS ring of its own (4 rows x 256 bytes, whole
    // 128-byte lines, per instruction; loaded straight into the fragment
    // registers one instruction covered 16 rows x 64 bytes): instruction j
    // of wave w fills its rows 4 j .. 4 j + 3 of weight d's stage; lane l
    // fills slot l % 16 of row 4 j + l / 16 from logical chunk (l % 16) ^
    // row, the swizzle of x.  Rows past n read row n - 1 (never stored);
    // bytes past the slice read its last 16 (masked in the tail).
    const int8_t *wsrc[D][4];
    int wcol[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + (lane >> 4);
        const int64_t wrow = min<int64_t>(n0 + r, p.n - 1) * p.k + k_lo;
        wsrc[0][j] = p.qw + wrow;
        if (DUAL) wsrc[D - 1][j] = p.qw2 + wrow;
        wcol[j] = 16 * ((lane & 15) ^ r);
    }
    const int kq = 16 * (lane >> 4);  // the lane's k offset within a step
    auto issue_w = [&](int i, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            int8_t *stage = wsm + slot * kWStageBytes + (d * kWaves + wave) * 16 * kChunk;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                __builtin_amdgcn_global_load_lds((glb_ptr)(wsrc[d][j] + min(i * kChunk + wcol[j], kl - 16)),
                                                 (lds_ptr)(stage + 4 * j * kChunk), 16, 0, kNtHint);
        }
    };

    i32x4 acc[D][MB];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[d][mb] = i32x4{0, 0, 0, 0};
    // Fragment of x block mb, step s: row 16 mb + l % 16, logical chunk
    // 4 s + l / 16.
    // The weight fragment is the same slot of row l % 16 of the wave's rows
    // in weight d's stage.
    const int xrd = (lane & 15) * kChunk;
    auto compute = [&](int u, auto tail, int i) __attribute__((always_inline)) {
        const int8_t *stage = xs + u * kStageBytes;
        const int8_t *wstage = wsm + u * kWStageBytes + wave * 16 * kChunk + xrd;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            i32x4 xv[MB], wv[D];
            const int sw = ((4 * s + (lane >> 4)) ^ (lane & 15)) << 4;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                xv[mb] = *reinterpret_cast<const i32x4 *>(stage + mb * 16 * kChunk + xrd + sw);
#pragma unroll
            for (int d = 0; d < D; ++d)
                wv[d] = *reinterpret_cast<const i32x4 *>(wstage + d * kWaves * 16 * kChunk + sw);
            if constexpr (decltype(tail)::value) {
                // K % 16 == 0: a lane's 16 bytes are all inside the slice or
                // all past it; past it both operands are zero.
                const bool ok = i * kChunk + 64 * s + kq < kl;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
#pragma unroll
                    for (int d = 0; d < D; ++d) wv[d][e] = ok ? wv[d][e] : 0;
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) xv[mb][e] = ok ? xv[mb][e] : 0;
                }
            }
#pragma unroll
            for (int d = 0; d < D; ++d)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[d][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xv[mb], wv[d], acc[d][mb], 0, 0, 0);
        }
    };

    // Chunk i (ring stage u = i % kStages): wait for its x and W (the next
    // chunk's loads stay in flight), barrier (its x is visible, and every
    // wave is done with chunk i - 1, whose stages now refill), issue chunk
    // i + 2 (unconditionally: past the last chunk it repeats the last one
    // into the free stages, so the wait count is one constant), compute
    // chunk i.
    const bool ragged = (kl % kChunk) != 0;
    auto step = [&](int i, int u) __attribute__((always_inline)) {
        wait_vmcnt<kOps>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int nx = min(i + 2, nch - 1);
        issue_x(nx, (u + 2) % kStages);
        __builtin_amdgcn_sched_barrier(0);  // x before W
        issue_w(nx, (u + 2) % kStages);
        __builtin_amdgcn_sched_barrier(0);
        if (ragged && i + 1 == nch)
            compute(u, std::true_type{}, i);
        else
            compute(u, std::false_type{}, i);
    };
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        issue_x(min(c, nch - 1), c);
        __builtin_amdgcn_sched_barrier(0);
        issue_w(min(c, nch - 1), c);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Whole rounds of three chunks (stage indices known at compile time),
    // then the one or two left.
    int i = 0;
    for (; i + kStages <= nch; i += kStages) {
#pragma unroll
        for (int u = 0; u < kStages; ++u) step(i + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < kStages; ++u)
        if (i + u < nch) step(i + u, u);
    wait_vmcnt<0>();          // no load may still be writing the ring
    if (n0 >= p.n) return;  // a wave past the last column (after every barrier)

    // 16x16 accumulator layout: lane l, register r -> row 4 (l / 16) + r of
    // the block, column l % 16.
    const int64_t col = n0 + (lane & 15);
    const bool col_ok = col < p.n;
    const int64_t blk = n0 / 16;
    auto row_of = [&](int mb, int r) -> int64_t { return (int64_t)mb * 16 + 4 * (lane >> 4) + r; };
    auto corrected = [&](int d, int64_t row, int32_t raw) -> int32_t {
        if (!p.zx) return raw;
        const int32_t *rs = d ? p.rowsum2 : p.rowsum;
        return (int32_t)((uint32_t)raw - (uint32_t)((int32_t)p.zx[p.x_per_row ? row : 0] * rs[col]));
    };
    auto dequant = [&](int d, int64_t row, int32_t a) -> float {
        const float *sw = d ? p.sw2 : p.sw;
        const float *bias = d ? p.bias2 : p.bias;
        const float sc = p.sx[p.x_per_row ? row : 0] * sw[col];
        float v = (float)a * sc;
        if (bias) v = v + bias[col];
        return v;
    };
    float mn = INFINITY, mx = -INFINITY;
    auto epilogue = [&](int64_t row, const int32_t *raw) {
        if (DUAL) {
            const float g = dequant(0, row, corrected(0, row, raw[0]));
            const float u = dequant(1, row, corrected(1, row, raw[D - 1]));
            const float h = silu_mul1(g, u);
            p.y[row * p.n + col] = h;
            mn = fminf(mn, h);
            mx = fmaxf(mx, h);
            return;
        }
        const int32_t a = corrected(0, row, raw[0]);
        if (p.acc) p.acc[row * p.n + col] = a;
        if (p.y) p.y[row * p.n + col] = dequant(0, row, a);
    };
    auto publish_minmax = [&]() {
        if (!DUAL) return;
        wave_minmax(mn, mx);
        if (lane == 0) p.hpart[blk] = make_float2(mn, mx);
    };

    if (sp.slices == 1) {
        if (col_ok) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = row_of(mb, r);
                    int32_t raw[D];
#pragma unroll
                    for (int d = 0; d < D; ++d) raw[d] = acc[d][mb][r];
                    if (row < p.m) epilogue(row, raw);
                }
        }
        publish_minmax();
        return;
    }

    // Publish the partial block with agent-scope stores (they go to the
    // device coherence point, so no cache writeback is needed), wait for
    // them, then count this wave's arrival on its column block.
    if (col_ok) {
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = row_of(mb, r);
                    if (row < p.m)
                        __hip_atomic_store(sp.part + ((slice * D + d) * p.m + row) * p.n + col, acc[d][mb][r],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
    }
    // split-K arrival protocol (common.hpp): steps 2-4
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    wait_vmcnt<0>();
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(sp.counters + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (int)sp.slices - 1;
    last = __shfl(last, 0);
    if (!last) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // The partials of all the lane's outputs for kGroup slices at a time are
    // requested before any is added, so the loads overlap; integer sums are
    // exact (wrapping as int32) in any order.
    constexpr int kGroup = 32 / (4 * MB * D) > 0 ? 32 / (4 * MB * D) : 1;
    uint32_t sum[D][MB][4];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) sum[d][mb][r] = 0;
    for (int64_t j0 = 0; j0 < sp.slices; j0 += kGroup) {
        int32_t pv[kGroup][D][MB][4];
#pragma unroll
        for (int g = 0; g < kGroup; ++g)
#pragma unroll
            for (int d = 0; d < D; ++d)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = row_of(mb, r);
                        const bool ok = col_ok && row < p.m && j0 + g < sp.slices;
                        pv[g][d][mb][r] = ok ? __hip_atomic_load(sp.part + (((j0 + g) * D + d) * p.m + row) * p.n + col,
                                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                             : 0;
                    }
#pragma unroll
        for (int g = 0; g < kGroup; ++g)
#pragma unroll
            for (int d = 0; d < D; ++d)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sum[d][mb][r] += (uint32_t)pv[g][d][mb][r];
    }
    if (col_ok) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_of(mb, r);
                if (row >= p.m) continue;
                int32_t raw[D];
#pragma unroll
                for (int d = 0; d < D; ++d) raw[d] = (int32_t)sum[d][mb][r];
                epilogue(row, raw);
            }
    }
    publish_minmax();
    if (lane == 0) __hip_atomic_store(sp.counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K bytes per workgroup: all of K with at least 128 column groups (half
// the CUs), otherwise enough slices for about 256 workgroups, each at least
// 4 chunks, a multiple of the chunk.  At N = 4096 (64 groups), K = 11008,
// M = 8 / 16 / 32 / 64: 14.1 / 14.3 / 16.1 / 20.9 us with 4 slices against
// 15.9 / 16.3 / 19.5 / 27.6 with 8 (a 512 target) and 16.9 / 17.1 / 19.4 /
// 25.0 with 2; K = 14336, M = 16 / 48: 16.1 / 19.9 against 17.1 / 24.4.  At N = 11008 (172 groups), K = 4096,
// no split beat 2 / 3 / 4 slices at every M measured: M = 8 / 16 / 32 14.1 /
// 14.0 / 15.5 us against 14.9-17.6 / 15.2-18.2 / 18.1-21.5 (the gate/up form
// 22.4 / 22.5 / 24.9 against 25.0-27.8 / 25.7-27.7 / 29.4-33.8): the split
// tail costs more than half the CUs idle.
int64_t choose_kslice(int64_t ngrp, int64_t k) {
    const int64_t kc = (k + kChunk - 1) / kChunk * kChunk;
    if (ngrp >= 128) return kc;
    int64_t s = (256 + ngrp - 1) / ngrp;
    s = std::max<int64_t>(1, std::min<int64_t>(s, k / (4 * kChunk)));
    if (s == 1) return kc;
    const int64_t ks = (k + s - 1) / s;
    return (ks + kChunk - 1) / kChunk * kChunk;
}

template <bool DUAL>
int launch(const QParams &p, hipStream_t s, int *npart = nullptr) {
    constexpr int D = DUAL ? 2 : 1;
    Params sp{};
    sp.q = p;
    sp.ngrp = (p.n + kGroupCols - 1) / kGroupCols;
    sp.kslice = choose_kslice(sp.ngrp, p.k);
    sp.slices = (p.k + sp.kslice - 1) / sp.kslice;
    if (npart) *npart = (int)((p.n + 15) / 16);
    if (sp.slices > 1) {
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(int32_t) * (size_t)(sp.slices * D * p.m * p.n), &ws));
        sp.part = static_cast<int32_t *>(ws);
        GFH_TRY(stream_counters(s, (size_t)(sp.ngrp * kWaves), &sp.counters));
    }
    const dim3 grid((unsigned)(sp.ngrp * sp.slices)), block(64 * kWaves);
    if (p.m <= 16)
        hipLaunchKernelGGL((qlinear_skinny_lds_kernel<1, DUAL>), grid, block, 0, s, sp);
    else if (p.m <= 32)
        hipLaunchKernelGGL((qlinear_skinny_lds_kernel<2, DUAL>), grid, block, 0, s, sp);
    else if (p.m <= 48)
        hipLaunchKernelGGL((qlinear_skinny_lds_kernel<3, DUAL>), grid, block, 0, s, sp);
    else
        hipLaunchKernelGGL((qlinear_skinny_lds_kernel<4, DUAL>), grid, block, 0, s, sp);
    return check_launch(DUAL ? "qlinear_swiglu_i8 (skinny, shared x)" : "qlinear_i8 (skinny, shared x)");
}

}  // namespace skinny_lds

// Which skinny kernel serves 1 <= M <= 64.  The 16-column kernel re-reads x
// per wave (m / 16 times the weight bytes again); the shared-x kernel reads
// it once per workgroup.  Measured (us, 16-column / shared x): N = 11008,
// K = 4096: M = 8 14.2 / 14.1, 16 16.3 / 14.0, 32 22.9 / 15.5, gate/up M =
// 16 25.8 / 22.5, 32 33.2 / 24.9; N = 4096, K = 11008: M = 16 19.6 / 16.9,
// 32 28.7 / 19.7; N = 4096, K = 4096, M = 16 11.2 / 9.2.  At 2-4 rows the
// shared-x kernel (with its weight ring) also wins, except where it would
// split K and the 16-column kernel would not: M = 2 / 4, N = 11008, K =
// 4096 11.8 / 12.3 against 12.5 / 13.4 us; N = 4096, K = 11008 13.5 / 14.1
// against 14.9 / 17.4 us; but N = 4096, K = 4096 8.8 / 9.3 against 6.7 /
// 7.3 us; M = 1 the same way (N = 11008, K = 4096 11.6 against 12.0 us).
// Activations quantized in the kernel (the decode SwiGLU, the dynamic
// linear) take the 16-column kernel before this choice.
bool use_skinny_lds(int64_t m, int64_t n, int64_t k, bool dual) {
    (void)dual;
    if (m > 4) return true;
    const bool lds_splits = skinny_lds::choose_kslice((n + skinny_lds::kGroupCols - 1) / skinny_lds::kGroupCols, k) < k;
    const bool cols16_splits = skinny::choose_kslice((n + skinny::kCols - 1) / skinny::kCols, k) < k;
    return !(lds_splits && !cols16_splits);
}

}  // namespace

bool qlinear_qx_fits(int64_t m, int64_t n, int64_t k, bool partials) { return skinny::qx_fits(m, n, k, partials); }

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
    p.xf = d.xf;
    p.xpart = d.xpart;
    p.nxpart = d.nxpart;
    if (d.xf) {  // activations quantized in the kernel (qlinear_qx_fits)
        if (!aligned16(d.qw)) return set_error(GFH_INVALID_DATA, "qlinear_i8: in-kernel quantization needs aligned qw");
        return skinny::launch<false>(p, s);
    }
    if (d.m <= 64 && d.k % 16 == 0 && d.k > 0 && aligned16(d.qx) && aligned16(d.qw))
        return use_skinny_lds(d.m, d.n, d.k, false) ? skinny_lds::launch<false>(p, s) : skinny::launch<false>(p, s);
    // Direct-to-LDS tiles need 16-byte aligned rows (K % 64 == 0) and 32-bit
    // row offsets inside a tile (256 * K < 2^32).
    const bool ring_ok = d.k > 0 && d.k % 64 == 0 && d.k <= (int64_t(1) << 24) && aligned16(d.qx) && aligned16(d.qw);
    // 8 waves per workgroup (a 2 x 4 wave grid, two waves per SIMD): one
    // wave's MFMAs run while the other waits on LDS or a barrier.  Measured
    // against 4 waves: 4096^3 76.7 -> 69.5 us, 4096 x 11008 x 4096 234.7 ->
    // 209.4 us; at N = 11008, K = 4096: M = 768 74.8 -> 60.8 us (256 x 256),
    // M = 512 50.5 -> 42.5 us (128 x 128, two workgroups per CU), M = 256
    // 27.2 -> 25.6 us (128 x 128, one per CU with a 3-deep ring).
    if (ring_ok) {
        const bool bk128 = d.k % 128 == 0;
        if (d.m > 512)
            return bk128 ? big::launch_tiles<256, 256, 128, 3, 2, 2, 4>(p, s)
                         : big::launch_tiles<256, 256, 64, 4, 4, 2, 4>(p, s);
        if (!bk128) return big::launch_tiles<128, 128, 64, 4, 4, 2, 4>(p, s);
        // 64 < M <= 512: the largest tile that still gives about 160
        // workgroups (128 x 128, then 64 x 128, else 64 x 64 with 4 waves and
        // a 4-deep ring, two or three workgroups per CU).  Measured (us,
        // 128 x 128 / 64 x 128 / 64 x 64): M = 256, N = 4096, K = 11008 53.3 /
        // 40.1 / 27.9; M = 512, N = 4096, K = 4096 19.4 / 11.6 / 13.9; M =
        // 256, N = 4096, K = 4096 17.2 / 10.4 / 8.2; M = 256, N = 11008, K =
        // 4096 26.0 / 31.7 / 29.8; M = 128, N = 11008 24.0 / 19.1 / 21.8.
        auto tiles = [&](int64_t bm, int64_t bn) { return ((d.m + bm - 1) / bm) * ((d.n + bn - 1) / bn); };
        // Long K with few tiles: split K over workgroups so that the grid
        // is one round of 256 (int32 partials, exact; the last slice of a
        // tile adds them).  The fewest slices that fill the round: 64 x 64
        // tiles when they leave room for two, else 128 x 128 ones (a 64 x 64
        // split needs a round of 512, slower).  Measured on uniform random
        // codes (us, unsplit / split): M = 128, N = 4096, K = 11008 29.3 /
        // 23.0 (64 x 64 in 2; 128 x 128 in 8: 26.3); M = 256, N = 4096
        // (64 x 64 unsplit against 128 x 128 in 4): K = 11008 32.0 / 29.2,
        // K = 14336 40.3 / 34.5, but K = 8192 24.2 / 24.6 and K = 4096 13.5 /
        // 22.4 -- the last slice's reads of the others' 64 KB partials cost
        // what a shorter K no longer saves.  Grids of 512 (two 128 x 128
        // workgroups per CU with 2-stage rings, or one per CU in two rounds)
        // took 1.4-1.7x as long.
        if (d.k >= 8192) {
            const int64_t t64 = tiles(64, 64), t128 = tiles(128, 128);
            if (2 * t64 <= 256)
                return big::launch_tiles<64, 64, 128, 4, 4, 2, 2>(p, s, (int)(256 / t64));
            if (t128 <= 128 && d.k >= 10240)
                return big::launch_tiles<128, 128, 128, 3, 3, 2, 4>(p, s, (int)(256 / t128));
        }
        constexpr int64_t kFill = 160;
        if (tiles(128, 128) >= kFill)
            return tiles(128, 128) <= 256 ? big::launch_tiles<128, 128, 128, 3, 3, 2, 4>(p, s)
                                          : big::launch_tiles<128, 128, 128, 2, 2, 2, 4>(p, s);
        if (tiles(64, 128) >= kFill) return big::launch_tiles<64, 128, 128, 4, 4, 2, 2>(p, s);
        return big::launch_tiles<64, 64, 128, 4, 4, 2, 2>(p, s);
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

// ---- SwiGLU gate/up ------------------------------------------------------------
//
// Decode sizes (m <= 64) use the skinny kernel with two weight streams;
// larger m the direct-to-LDS tiles with gate and up rows interleaved in
// 32-row blocks: 128 x (64 + 64) up to m = 128, 256 x (64 + 64) up to 256
// (both a 4 x 2 wave grid, so that every wave holds both halves of its
// columns), 256 x (128 + 128) above.  Each workgroup takes one CU (its ring
// is 128-160 KB), so the tile is the one with the fewest operand bytes per
// CU over the whole launch: rounds of 256 workgroups x bytes per tile.  At
// N = 11008, K = 4096, m = 256 the 128-row tile needs two rounds of 1 MB
// (344 workgroups), the 256-row tile one round of 1.5 MB (172); at m = 512
// the 256 x 256 tile one round of 2 MB against three of 1 MB (688).

bool qlinear_swiglu_fits(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % 16 != 0) return false;
    if (m <= 64) return true;
    return k % 64 == 0 && k <= (int64_t(1) << 24);
}

int64_t qlinear_swiglu_partials(int64_t m, int64_t n) {
    if (m <= 64) return (n + skinny::kCols - 1) / skinny::kCols;
    if (m > 256) return ((m + 255) / 256) * ((n + 127) / 128);
    if (m > 128) return ((m + 255) / 256) * ((n + 63) / 64);
    return ((m + 127) / 128) * ((n + 63) / 64);
}

int launch_qlinear_swiglu_i8(const QSwigluDesc &d, int *npart, hipStream_t s) {
    const QLinearDesc &g = d.g;
    if (!qlinear_swiglu_fits(g.m, g.n, g.k) || g.x_per_row || !(g.xf || aligned16(g.qx)) || !aligned16(g.qw) ||
        !aligned16(d.qw_up))
        return set_error(GFH_INVALID_DATA, "qlinear_swiglu_i8: shape or alignment not served by the fused kernel");
    QParams p{};
    p.qx = g.qx;
    p.sx = g.sx;
    p.zx = g.zx;
    p.qw = g.qw;
    p.sw = g.sw;
    p.rowsum = g.w_rowsum;
    p.bias = g.bias;
    p.y = g.y;
    p.m = g.m;
    p.n = g.n;
    p.k = g.k;
    p.qw2 = d.qw_up;
    p.sw2 = d.sw_up;
    p.rowsum2 = d.rowsum_up;
    p.bias2 = d.bias_up;
    p.hpart = d.hpart;
    p.xf = g.xf;
    p.xpart = g.xpart;
    p.nxpart = g.nxpart;
    if (g.xf) return skinny::launch<true>(p, s, npart);  // activations quantized in the kernel
    if (g.m <= 64)
        return use_skinny_lds(g.m, g.n, g.k, true) ? skinny_lds::launch<true>(p, s, npart)
                                                    : skinny::launch<true>(p, s, npart);
    const bool bk128 = g.k % 128 == 0;
    if (g.m > 256)
        return bk128 ? big::launch_tiles_dual<256, 256, 128, 3, 2, 2, 4>(p, s, npart)
                     : big::launch_tiles_dual<256, 256, 64, 4, 4, 2, 4>(p, s, npart);
    if (g.m > 128)
        return bk128 ? big::launch_tiles_dual<256, 128, 128, 3, 3, 4, 2>(p, s, npart)
                     : big::launch_tiles_dual<256, 128, 64, 4, 4, 4, 2>(p, s, npart);
    // (a 4-deep ring: M = 128 / 256 / 512 at N = 11008, K = 4096 28.6 / 51.4
    // / 80.1 us against 29.2 / 54.1 / 85.2 with 3 on this tile; 64-row tiles
    // were slower)
    return bk128 ? big::launch_tiles_dual<128, 128, 128, 4, 4, 4, 2>(p, s, npart)
                 : big::launch_tiles_dual<128, 128, 64, 4, 4, 4, 2>(p, s, npart);
}

}  // namespace gfh
