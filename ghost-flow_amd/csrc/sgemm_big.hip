// sgemm_big.hip -- fp32 GEMM on 256 x 256, 128 x 128 or 64 x 64 tiles fed by
// direct-to-LDS loads:
// C = alpha * op(A) . op(B) (+ beta C) (+ bias) with A [m, k] or, transposed,
// [k, m] row-major and B either [n, k] (NT: Linear::forward's x . W^T with
// the reference's [out, in] weight, ghostflow-nn/src/linear.rs:56-69) or
// [k, n] (NN: Tensor::matmul, ghostflow-core/src/ops/matmul.rs:91-119).  The
// transposed A is matmul_backward's a^T . grad
// (ghostflow-autograd/src/backward.rs:131-160); a batch of such products
// runs as the grid's y dimension with batched_matmul's modulo slice indexing
// (matmul.rs:122-170).  gfh_sgemm and gfh_sgemm_strided_batched send those
// calls here when the problem fills the GPU with such tiles; the general
// tile kernel (sgemm.hip) serves everything else.
//
// Design (one 512-thread workgroup = 8 wave64s, 2 x 4, per 256 x 256 tile;
// 64 x 64 tiles run 2 x 2 waves twice over, as two wave sets that split
// every stage's k-groups and add their accumulators through LDS at the end):
//  * Each wave holds a 128 x 64 sub-tile as 4 x 2 v_mfma_f32_32x32x2_f32
//    accumulators (128 registers): 8 independent MFMA chains, and two waves
//    per SIMD so that one issues MFMAs while the other waits on LDS.
//  * K advances in stages of 32 floats (128 bytes per row).  Both operands
//    stream into a 2-stage LDS ring with global_load_lds_dwordx4 (global ->
//    LDS, no VGPR staging): one load instruction fills 1 KB = 8 rows x 128
//    bytes, whole cache lines.  Chunk c (16 bytes) of row r sits at
//    c ^ ((r >> 1) & 7), which puts the 16-byte fragment reads of 16 lanes
//    on 16 distinct 4-bank groups.
//  * Fragments: lane l reads row l % 32, chunk 2 kg + l / 32 of k-group kg
//    (8 floats): lanes 0-31 hold k 8kg .. 8kg+3, lanes 32-63 8kg+4 .. +7, and
//    element e of both operands feeds MFMA e of the group, so every product
//    pairs matching k.  The next group's fragments are read while the
//    current group's MFMAs run.
//  * NN: the B stage is 32 k-rows of 256 columns; one load instruction
//    fills one k-row (1 KB).  Rows sit 264 floats apart, so the B fragment
//    -- 4 scalar reads of 4 consecutive k for column l % 32 -- puts lanes
//    0-31 and 32-63 (4 rows apart) on disjoint halves of the 64 banks.  A
//    transposed A is staged and read the same way, in k-rows of the tile's
//    C rows.
//  * The loop body is branch-free: past the end of K the ring reloads the
//    last stage into the slot just freed, so every s_waitcnt is a constant.
//  * Epilogue: alpha * acc (+ beta C) (+ bias), separate f32 roundings as in
//    the reference; the tile goes through LDS so each wave stores whole
//    row runs with 16-byte stores.
//  * Workgroups are renumbered XCD-contiguous and walked in 4-tile bands so
//    tiles running together share A / B panels in one L2.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int BKB = 128;                  // K bytes per stage (32 floats)
constexpr int kRowsPerLoad = 1024 / BKB;  // K-contiguous rows per load instruction
constexpr int kGroupM = 4;
constexpr int kKGroups = BKB / 32;  // 8-float k-groups per stage

// Geometry of a BM x BN tile on an NWM_ x NWN_ wave grid with an
// STAGES_-deep ring: 256 x 256 and 128 x 128 on 2 x 4 waves and 2 stages,
// 64 x 64 on 2 x 2 waves and 4 stages.
template <int BM, int BN, bool NN, int NWM_ = 2, int NWN_ = 4, int STAGES_ = 2, int KS_ = 1, bool TA_ = false>
struct Geo {
    // KS wave sets share the tile: set s computes k-groups [s kKGroups / KS,
    // (s + 1) kKGroups / KS) of every stage into its own accumulators, which
    // are added through LDS at the end -- KS waves per SIMD on a tile that
    // has one wave per SIMD otherwise.
    static constexpr int KS = KS_;
    static_assert(KS == 1 || KS == 2, "wave sets");
    static constexpr int NWM = NWM_, NWN = NWN_, NW = NWM * NWN;  // tile wave grid
    static constexpr int NWT = NW * KS, NT = 64 * NWT;            // waves, threads
    static constexpr int STAGES = STAGES_;
    static constexpr int WM = BM / NWM, WN = BN / NWN;  // wave sub-tile
    static constexpr int FM = WM / 32, FN = WN / 32;    // accumulators per wave
    // load instructions (1 KB each) per wave per stage, over all NWT waves
    static constexpr int kLA = BM * BKB / (1024 * NWT), kLB = BN * BKB / (1024 * NWT);
    static_assert(kLA * 1024 * NWT == BM * BKB && kLB * 1024 * NWT == BN * BKB, "whole load instructions per wave");
    static constexpr int kLPS = kLA + kLB;
    // NN: a load instruction fills RPL k-rows of BN floats (1 KB); groups
    // of RPL rows sit 1024 + 32 RPL bytes apart, which puts rows 4 apart
    // 32 banks apart.  A transposed A ([k, m] in memory, TA) is staged the
    // same way, in k-rows of BM floats.
    static constexpr bool TA = TA_;
    static constexpr int RPL = 1024 / (BN * 4);
    static constexpr int kGroupStride = 1024 + 32 * RPL;
    static constexpr int RPLA = 1024 / (BM * 4);
    static constexpr int kGroupStrideA = 1024 + 32 * RPLA;
    static constexpr int kABytes = TA ? (32 / RPLA) * kGroupStrideA : BM * BKB;
    static constexpr int kBBytes = NN ? (32 / RPL) * kGroupStride : BN * BKB;
    static constexpr int kStageBytes = kABytes + kBBytes;
    static constexpr int kOutStride = WN + 8;  // floats per staged output row
    // The output goes through LDS half a wave sub-tile at a time, all of it
    // when the sub-tile is a single 32-row block.
    static constexpr int kOutPasses = FM >= 2 ? 2 : 1;
    static constexpr int kOutRows = WM / kOutPasses;
    static constexpr int kOut = NW * kOutRows * kOutStride * 4;
    static constexpr int kLds = STAGES * kStageBytes > kOut ? STAGES * kStageBytes : kOut;
    static_assert(kLds <= 160 * 1024, "LDS per workgroup");
    static_assert(KS == 1 || NW * FM * FN * 16 * 64 * 4 <= kLds, "accumulator exchange fits the ring");
    static_assert(FM >= 1 && FN >= 1 && (FM == 1 || FM % 2 == 0), "wave sub-tile");
    static_assert((STAGES - 1) * kLPS < 64, "vmcnt is 6 bits");
    // byte offset of k-row r inside an NN B stage / a TA A stage
    static __device__ __forceinline__ int brow(int r) { return (r / RPL) * kGroupStride + (r % RPL) * BN * 4; }
    static __device__ __forceinline__ int arow(int r) { return (r / RPLA) * kGroupStrideA + (r % RPLA) * BM * 4; }
};

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(1))) void *glb_ptr;

struct BigParams {
    const float *a, *b;
    float *c;
    const float *bias;
    int64_t m, n, k, lda, ldb, ldc;
    // batch z (blockIdx.y) takes A slice z % batch_a and B slice z % batch_b
    // (batched_matmul's modulo indexing) and writes C slice z
    int64_t stride_a, stride_b, stride_c;
    int batch_a, batch_b;
    float alpha, beta;
    int tiles_m, tiles_n;
    // split K (unbatched): workgroup z * tiles + t computes tile t over
    // stages [z kslice, (z + 1) kslice) of 32 k; each slice publishes its
    // partial tile in part and the last to arrive sums all slices in slice
    // order and runs the epilogue
    int slices, kslice;
    float *part;
    int *counters;
};

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// NM MFMAs with ND LDS reads and NV global loads spread between them.
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

template <int BM, int BN, bool NN, int NWM_ = 2, int NWN_ = 4, int STAGES_ = 2, int KS_ = 1, bool TA = false,
          bool BATCH = false>
__global__ __launch_bounds__((Geo<BM, BN, NN, NWM_, NWN_, STAGES_, KS_, TA>::NT),
                             (BM * BN <= 128 * 128) ? 2 : 1) void sgemm_big_kernel(BigParams p) {
    using G = Geo<BM, BN, NN, NWM_, NWN_, STAGES_, KS_, TA>;
    constexpr int NWN = G::NWN, NW = G::NW, NWT = G::NWT, STAGES = G::STAGES, KS = G::KS;
    constexpr int KGP = kKGroups / KS;  // k-groups per stage of this wave's set
    constexpr int WM = G::WM, WN = G::WN, FM = G::FM, FN = G::FN;
    constexpr int kLA = G::kLA, kLB = G::kLB, kLPS = G::kLPS;
    constexpr int kABytes = G::kABytes, kStageBytes = G::kStageBytes, kOutStride = G::kOutStride;
    __shared__ __attribute__((aligned(1024))) char lds[G::kLds];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0 .. NWT - 1: loads
    const int wt = wave % NW;                                     // position in the tile
    const int ks = wave / NW;                                     // wave set
    const int kg0 = ks * KGP;                                     // its first k-group of a stage
    const int wm0 = (wt / NWN) * WM;
    const int wn0 = (wt % NWN) * WN;

    const int nblk = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    int slice = 0;
    if (!BATCH && p.slices > 1) {
        slice = bid / nblk;
        bid -= slice * nblk;
    }
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int group_size = kGroupM * p.tiles_n;
    const int group = bid / group_size;
    const int first_m = group * kGroupM;
    const int gm = min(p.tiles_m - first_m, kGroupM);
    const int in_group = bid - group * group_size;
    const int64_t m0 = (int64_t)(first_m + in_group % gm) * BM;
    const int64_t n0 = (int64_t)(in_group / gm) * BN;
    const float *pa = p.a, *pb = p.b;
    float *pc = p.c;
    if constexpr (BATCH) {
        const int bz = blockIdx.y;
        pa += (bz % p.batch_a) * p.stride_a;
        pb += (bz % p.batch_b) * p.stride_b;
        pc += bz * p.stride_c;
    }

    // Byte offsets, from the tile's first row, of this wave's load
    // instructions: instruction j covers tile rows wave * (BM / NW) + j * 8
    // .. + 7; lane l fills LDS slot l of that 1 KB run (row l / 8, chunk
    // l % 8) from logical chunk (l % 8) ^ swz(row).  Rows past m / n read
    // the last row (their products are never stored).
    const int64_t k_lo = (int64_t)slice * p.kslice * 32;  // first k of this workgroup's slice
    const char *a_base = reinterpret_cast<const char *>(TA ? pa + k_lo * p.lda + m0 : pa + m0 * p.lda + k_lo);
    const char *b_base = reinterpret_cast<const char *>(NN ? pb + k_lo * p.ldb + n0 : pb + n0 * p.ldb + k_lo);
    int64_t a_off[kLA], b_off[kLB];
#pragma unroll
    for (int j = 0; j < kLA; ++j) {
        if (TA) {
            // row group wave * kLA + j: k-row RPLA g + l / (64 / RPLA), rows
            // m0 + 4 (l % (64 / RPLA)) .. + 3 of C (clamped below m; m % 4 == 0)
            constexpr int LPRA = 64 / G::RPLA;
            const int kr = (wave * kLA + j) * G::RPLA + lane / LPRA;
            a_off[j] = (int64_t)kr * p.lda * 4 + (min(m0 + 4 * (lane % LPRA), p.m - 4) - m0) * 4;
        } else {
            const int r = wave * (BM / NWT) + j * kRowsPerLoad + lane / 8;
            a_off[j] = (min(m0 + r, p.m - 1) - m0) * p.lda * 4 + ((lane % 8) ^ swz(r)) * 16;
        }
    }
#pragma unroll
    for (int j = 0; j < kLB; ++j) {
        if (NN) {
            // row group wave * kLB + j: k-row RPL g + l / (64 / RPL), columns
            // n0 + 4 (l % (64 / RPL)) .. + 3 (clamped below n; n % 4 == 0, so a
            // lane's 4 are all valid)
            constexpr int LPR = 64 / G::RPL;
            const int kr = (wave * kLB + j) * G::RPL + lane / LPR;
            b_off[j] = (int64_t)kr * p.ldb * 4 + (min(n0 + 4 * (lane % LPR), p.n - 4) - n0) * 4;
        } else {
            const int r = wave * (BN / NWT) + j * kRowsPerLoad + lane / 8;
            b_off[j] = (min(n0 + r, p.n - 1) - n0) * p.ldb * 4 + ((lane % 8) ^ swz(r)) * 16;
        }
    }
    // bytes between consecutive stages of A / B in global memory
    const int64_t a_stage = TA ? (int64_t)32 * p.lda * 4 : BKB;
    const int64_t b_stage = NN ? (int64_t)32 * p.ldb * 4 : BKB;
    const int nk = (int)min((int64_t)p.kslice, p.k / 32 - (int64_t)slice * p.kslice);

    auto issue = [&](int t, int slot) __attribute__((always_inline)) {
        char *la = lds + slot * kStageBytes;
        char *lb = la + kABytes;
#pragma unroll
        for (int j = 0; j < kLA; ++j) {
            char *dst = TA ? la + (wave * kLA + j) * G::kGroupStrideA : la + (wave * (BM / NWT) + j * kRowsPerLoad) * BKB;
            __builtin_amdgcn_global_load_lds((glb_ptr)(a_base + (int64_t)t * a_stage + a_off[j]), (lds_ptr)dst, 16, 0,
                                             0);
        }
#pragma unroll
        for (int j = 0; j < kLB; ++j) {
            char *dst = NN ? lb + (wave * kLB + j) * G::kGroupStride : lb + (wave * (BN / NWT) + j * kRowsPerLoad) * BKB;
            __builtin_amdgcn_global_load_lds((glb_ptr)(b_base + (int64_t)t * b_stage + b_off[j]), (lds_ptr)dst, 16, 0,
                                             0);
        }
    };

    // Fragment of k-group kg: lane l reads row l % 32 of a 32-row block,
    // logical chunk 2 kg + l / 32; blocks start at multiples of 32 rows, so
    // the swizzle depends on the lane only.
    const int frow = lane & 31;
    const int foff0 = frow * BKB + (((lane >> 5) ^ swz(frow)) * 16);
    f32x4 af[2][FM], bf[2][FN];
    auto load_frags = [&](int buf, int t, int kg) __attribute__((always_inline)) {
        const char *la = lds + (t % STAGES) * kStageBytes;
        const char *lb = la + kABytes;
        const int fo = foff0 ^ (kg << 5);
        if (TA) {
            const int r0 = 8 * kg + 4 * (lane >> 5);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float *fa = reinterpret_cast<const float *>(la + G::arow(r0 + e)) + (lane & 31);
#pragma unroll
                for (int i = 0; i < FM; ++i) af[buf][i][e] = fa[wm0 + i * 32];
            }
        } else {
#pragma unroll
            for (int i = 0; i < FM; ++i) af[buf][i] = *reinterpret_cast<const f32x4 *>(la + (wm0 + i * 32) * BKB + fo);
        }
        if (NN) {
            const int r0 = 8 * kg + 4 * (lane >> 5);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float *fb = reinterpret_cast<const float *>(lb + G::brow(r0 + e)) + (lane & 31);
#pragma unroll
                for (int j = 0; j < FN; ++j) bf[buf][j][e] = fb[wn0 + j * 32];
            }
        } else {
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[buf][j] = *reinterpret_cast<const f32x4 *>(lb + (wn0 + j * 32) * BKB + fo);
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    auto mfmas = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[buf][i][e], bf[buf][j][e], acc[i][j], 0, 0, 0);
    };

    constexpr int NR = (TA ? 4 : 1) * FM + (NN ? 4 : 1) * FN, NM = 4 * FM * FN;
    for (int t = 0; t < STAGES; ++t) issue(min(t, nk - 1), t);
    wait_vmcnt<(STAGES - 1) * kLPS>();
    __builtin_amdgcn_s_barrier();
    load_frags(0, 0, kg0);
    // (inlined: a call would pass the accumulators through scratch memory)
    auto k_groups = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u + 1 < KGP; ++u) {
            load_frags((u + 1) & 1, t, kg0 + u + 1);
            mfmas(u & 1);
            interleave<0, NR, NM>();
        }
    };
    for (int t = 0; t + 1 < nk; ++t) {
        k_groups(t);
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkm0();  // this wave's reads of stage t are done
        wait_vmcnt<(STAGES - 2) * kLPS>();  // stage t + 1 landed
        __builtin_amdgcn_s_barrier();
        issue(min(t + STAGES, nk - 1), t % STAGES);
        load_frags(0, t + 1, kg0);
        mfmas((KGP - 1) & 1);
        interleave<kLPS, NR, NM>();
        __builtin_amdgcn_sched_barrier(0);
    }
    k_groups(nk - 1);
    mfmas((KGP - 1) & 1);
    wait_vmcnt<0>();  // no load may still be writing the ring

    if constexpr (KS == 2) {
        // set 1 hands its accumulators to set 0 through the idle ring; set 0
        // adds them (set 0 + set 1, a fixed order) and writes the tile
        __syncthreads();
        float *xch = reinterpret_cast<float *>(lds) + wt * (FM * FN * 16 * 64) + lane;
        if (ks == 1) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) xch[((i * FN + j) * 16 + r) * 64] = acc[i][j][r];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] + xch[((i * FN + j) * 16 + r) * 64];
        }
    }

    if (!BATCH && p.slices > 1) {
        // Split K.  Every slice publishes its tile (register quad q of
        // thread t at [slot][q][t]: 16-byte stores and loads, coalesced, at
        // the device coherence point) and counts its arrival (the split-K
        // protocol of common.hpp); the last to arrive sums all slices'
        // partials in slice order, so the result does not depend on the
        // order of arrival.  With two wave sets the tile is in set 0.
        constexpr int R4 = FM * FN * 4, NTP = NW * 64;
        const uint32_t part_bytes = (uint32_t)((int64_t)p.slices * nblk * R4 * NTP * 16);
        const __amdgpu_buffer_rsrc_t part_buf = coherent_buffer(p.part, part_bytes);
        const int tp = wt * 64 + lane;
        auto part_off = [&](int sl, int q) { return (uint32_t)((((int64_t)sl * nblk + bid) * R4 + q) * NTP + tp) * 16; };
        if (KS == 1 || ks == 0) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), part_buf,
                                                               part_off(slice, (i * FN + j) * 4 + q), 0, kScDevice);
                    }
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        wait_vmcnt<0>();  // this thread's partial stores are complete
        __syncthreads();  // (the flag goes through the idle ring)
        int *last_flag = reinterpret_cast<int *>(lds);
        if (tid == 0)
            *last_flag =
                __hip_atomic_fetch_add(p.counters + bid, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.slices - 1;
        __syncthreads();
        if (!*last_flag) return;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (KS == 1 || ks == 0) {
            // slice 0 + slice 1 + ..., a block of 4 registers at a time with
            // every slice's load of it requested before the first add
            constexpr int GS = 8;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int qq = (i * FN + j) * 4 + q;
                        f32x4 tot = {0.f, 0.f, 0.f, 0.f};
                        for (int s0 = 0; s0 < p.slices; s0 += GS) {
                            i32x4 t[GS];
#pragma unroll
                            for (int g = 0; g < GS; ++g)
                                t[g] = s0 + g < p.slices
                                           ? __builtin_amdgcn_raw_buffer_load_b128(part_buf, part_off(s0 + g, qq), 0,
                                                                                   kScDevice)
                                           : i32x4{0, 0, 0, 0};
#pragma unroll
                            for (int g = 0; g < GS; ++g) {
                                const f32x4 v = __builtin_bit_cast(f32x4, t[g]);
                                if (s0 + g == 0)
                                    tot = v;
                                else if (s0 + g < p.slices)
                                    tot = tot + v;
                            }
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] = tot[e];
                    }
        }
        if (tid == 0) __hip_atomic_store(p.counters + bid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Epilogue.  Lane l, register r of block (i, j): row 8 (r / 4) +
    // 4 (l / 32) + r % 4, column l % 32.  Each wave converts half of its
    // sub-tile at a time into its own LDS region, then writes whole row
    // runs of WN floats with 16-byte stores.
    constexpr int LPR = WN / 4;    // lanes per output row
    constexpr int RPI = 64 / LPR;  // rows per store instruction
    constexpr int PASSES = G::kOutPasses;
    constexpr int HALF = G::kOutRows;  // rows per pass
    constexpr int BPP = FM / PASSES;   // 32-row blocks per pass
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();  // every wave is done with the operand ring
    float *lt = reinterpret_cast<float *>(lds) + wt * (HALF * kOutStride);
    const bool vec_out = (p.ldc % 4) == 0 && (reinterpret_cast<uintptr_t>(pc) & 15) == 0;
#pragma unroll
    for (int hf = 0; hf < PASSES; ++hf) {
        if (KS == 1 || ks == 0) {  // (set 1 only keeps the barriers)
#pragma unroll
            for (int ii = 0; ii < BPP; ++ii)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int lr = ii * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        lt[lr * kOutStride + j * 32 + (lane & 31)] = p.alpha * acc[hf * BPP + ii][j][r];
                    }
            const int64_t col = n0 + wn0 + 4 * (lane % LPR);
#pragma unroll
            for (int q = 0; q < HALF / RPI; ++q) {
                const int lr = RPI * q + lane / LPR;
                f32x4 v = *reinterpret_cast<const f32x4 *>(lt + lr * kOutStride + 4 * (lane % LPR));
                const int64_t row = m0 + wm0 + hf * HALF + lr;
                if (row >= p.m) continue;
                float *dst = pc + row * p.ldc + col;
                if (vec_out && col + 3 < p.n) {
                    if (p.beta != 0.f) {
                        const f32x4 c0 = *reinterpret_cast<const f32x4 *>(dst);
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = v[e] + p.beta * c0[e];
                    }
                    if (p.bias) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = v[e] + p.bias[col + e];
                    }
                    *reinterpret_cast<f32x4 *>(dst) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (col + e >= p.n) continue;
                        float x = v[e];
                        if (p.beta != 0.f) x = x + p.beta * dst[e];
                        if (p.bias) x = x + p.bias[col + e];
                        dst[e] = x;
                    }
                }
            }
        }
        __builtin_amdgcn_s_barrier();  // the region is refilled by the next half
    }
}

}  // namespace

namespace {
// output tiles of side t over the whole batch
int64_t tiles_of(const SgemmDesc &d, int64_t t) { return ((d.m + t - 1) / t) * ((d.n + t - 1) / t) * d.batch; }

// One tile configuration in the four operand layouts (A as [m, k] or, with
// trans_a, [k, m]; B as [k, n] or, with trans_b, [n, k]); batched products
// take A as [m, k].
template <int BM, int BN, int NWM, int NWN, int STAGES, int KS>
void launch_layouts(bool trans_a, bool trans_b, bool batched, const BigParams &p, dim3 grid, hipStream_t s) {
    constexpr int kThreads = Geo<BM, BN, false, NWM, NWN, STAGES, KS>::NT;
    const dim3 block(kThreads);
    if (batched) {
        if (trans_b)
            hipLaunchKernelGGL((sgemm_big_kernel<BM, BN, false, NWM, NWN, STAGES, KS, false, true>), grid, block, 0, s,
                               p);
        else
            hipLaunchKernelGGL((sgemm_big_kernel<BM, BN, true, NWM, NWN, STAGES, KS, false, true>), grid, block, 0, s,
                               p);
    } else if (trans_a) {
        if (trans_b)
            hipLaunchKernelGGL((sgemm_big_kernel<BM, BN, false, NWM, NWN, STAGES, KS, true>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((sgemm_big_kernel<BM, BN, true, NWM, NWN, STAGES, KS, true>), grid, block, 0, s, p);
    } else {
        if (trans_b)
            hipLaunchKernelGGL((sgemm_big_kernel<BM, BN, false, NWM, NWN, STAGES, KS, false>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((sgemm_big_kernel<BM, BN, true, NWM, NWN, STAGES, KS, false>), grid, block, 0, s, p);
    }
}
}  // namespace

// Whether these tiles take the product: at least 256 tiles of 128 x 128 or
// 32 of 64 x 64 (counting every batch slice), or, unbatched, 16 or more rows
// with K >= 1024 and at least 16 tiles of 64 x 64 (split K then fills the
// CUs).  launch_sgemm_big picks the tile size and the K split.
// Measured against the register-staged tile kernel (us): 1024^3 NN 31.3 ->
// 25.8, NT 29.5 -> 20.9; 1536^3 NN 120.5 -> 84.4; 1024 x 1024 x 4096 NN
// 107.2 -> 86.6; 512 x 2048 x 1024 NT 29.5 -> 20.7.
bool sgemm_big_fits(const SgemmDesc &d) {
    if (d.k <= 0 || d.k % 32 != 0 || d.lda % 4 != 0 || d.ldb % 4 != 0) return false;
    if (!d.trans_b && d.n % 4 != 0) return false;  // B as [k, n]: whole 16-byte column groups
    if (d.trans_a && d.m % 4 != 0) return false;   // A as [k, m]: the same
    if (!aligned16(d.a) || !aligned16(d.b)) return false;
    if (d.batch > 1 || d.batch_a > 1 || d.batch_b > 1) {
        // A as [m, k]; every slice 16-byte aligned; the batch is the grid's
        // y dimension
        if (d.trans_a || d.stride_a % 4 != 0 || d.stride_b % 4 != 0 || d.batch > 65535) return false;
    }
    if (d.m >= 128 && d.n >= 128 && tiles_of(d, 128) >= 256) return true;
    if (d.m >= 64 && d.n >= 64 && tiles_of(d, 64) >= 32) return true;
    // A few rows of an unbatched product with a long K: 64 x 64 tiles with K
    // split over the CUs (split_k_slices).
    return d.batch <= 1 && d.batch_a <= 1 && d.batch_b <= 1 && d.m >= 16 && d.n >= 64 && d.k >= 1024 &&
           tiles_of(d, 64) >= 16;
}

namespace {
// K slices for an unbatched launch of `tiles` workgroups over `stages`
// stages of 32 k: enough to bring a launch of fewer than 256 tiles to about
// one workgroup per CU, at most 8, each slice at least 8 stages.
int split_k_slices(int64_t tiles, int64_t stages) {
    if (tiles >= 256) return 1;
    int64_t sl = std::min<int64_t>(std::min<int64_t>(8, 256 / std::max<int64_t>(tiles, 1)), stages / 8);
    return (int)std::max<int64_t>(sl, 1);
}
}  // namespace

int launch_sgemm_big(const SgemmDesc &d, hipStream_t s) {
    BigParams p{};
    p.a = d.a;
    p.b = d.b;
    p.c = d.c;
    p.bias = d.bias;
    p.m = d.m;
    p.n = d.n;
    p.k = d.k;
    p.lda = d.lda;
    p.ldb = d.ldb;
    p.ldc = d.ldc;
    p.stride_a = d.stride_a;
    p.stride_b = d.stride_b;
    p.stride_c = d.stride_c;
    // (a slice count above the batch indexes like the batch itself)
    const int64_t nb = std::max<int64_t>(d.batch, 1);
    p.batch_a = (int)std::min(std::max<int64_t>(d.batch_a, 1), nb);
    p.batch_b = (int)std::min(std::max<int64_t>(d.batch_b, 1), nb);
    const bool batched = d.batch > 1 || d.batch_a > 1 || d.batch_b > 1;
    p.alpha = d.alpha;
    p.beta = d.beta;
    // 256 x 256 tiles need K >= 256: below that a tile's epilogue outweighs
    // its K loop, and 128 x 128 tiles, two workgroups per CU, overlap one
    // tile's stores with the other's loop (batched 512 x 512 x 128 slices,
    // 128 of them: 89.0 -> 85.8 us; 2048 x 2048 x 128: 1341 -> 1308 us).
    // Between 256 x 256 and 128 x 128 tiles, the one with the shorter
    // estimated time, in units of a 256 x 256 tile's K loop (one round of
    // 256 of them): a round of 512 tiles of 128 x 128, two per CU, takes
    // 0.54 of it (4096^3: 1001 against 930 us for twice the rounds), and up
    // to 256 of them, one per CU, 0.28 (2048^3: 131 us at K = 2048).  The
    // larger tile keeps near-ties.  Measured at N = 14336, K = 4096 (us):
    // M = 768 747 on 128 x 128 (930 on 256 x 256), M = 1024 932 on 256 x 256
    // (990), M = 1536 1492 on 128 x 128 (1852).
    const int64_t t128 = tiles_of(d, 128), t256 = tiles_of(d, 256);
    const bool ok256 = d.m >= 256 && d.n >= 256 && d.k >= 256;
    const bool ok128 = d.m >= 128 && d.n >= 128 && t128 >= 256;
    const double r256 = (double)((t256 + 255) / 256);
    const int64_t rem128 = t128 % 512;
    const double r128 = t128 <= 256 ? 0.28
                                    : 0.54 * (double)(t128 / 512) + (rem128 == 0 ? 0.0 : rem128 <= 256 ? 0.28 : 0.54);
    int t = (ok256 && (!ok128 ? t256 >= 256 : r128 >= 0.95 * r256)) ? 256 : ok128 ? 128 : 64;
    // 32-255 tiles of 128 x 128 over a long K, with K split (split_k_slices),
    // where they fill half again as many CUs as the 64 x 64 tiles do (768 x
    // 768 x 8192: 252 workgroups of 128 x 128 against 144 of 64 x 64, 85.7
    // against 147 us; where both fill the GPU, as at 1024 x 1024 x 4096,
    // either tile takes 70-77 us).
    if (t == 64 && !batched && d.m >= 128 && d.n >= 128 && t128 >= 32 && d.k >= 1024) {
        const int64_t t64 = tiles_of(d, 64), stages = d.k / 32;
        if (2 * t128 * split_k_slices(t128, stages) >= 3 * t64 * split_k_slices(t64, stages)) t = 128;
    }
    // Up to 32 rows of an unbatched product: 32 x 64 tiles (two wave sets
    // of 1 x 2 waves), so that half of each MFMA's rows is not padding.
    const int tm = (t == 64 && !batched && d.m <= 32) ? 32 : t;
    p.tiles_m = (int)((d.m + tm - 1) / tm);
    p.tiles_n = (int)((d.n + t - 1) / t);
    const int64_t nblk = (int64_t)p.tiles_m * p.tiles_n, stages = d.k / 32;
    p.slices = 1;
    p.kslice = (int)stages;
    if (!batched) {
        int sl = split_k_slices(nblk, stages);
        if (t == 128 && nblk > 256) {
            // 128 x 128 tiles two per CU: the slice count (up to 4) with the
            // shortest estimated time in the rounds model above, plus 0.03
            // for publishing and summing partial tiles (N = 14336, K = 4096:
            // M = 384, 336 tiles in 3 slices, 492 -> 340 us; M = 640, 560
            // tiles in 4 slices, 736 -> 572 us)
            double best = 1e30;
            for (int c = 1; c <= 4 && stages / c >= 8; ++c) {
                const int64_t tasks = nblk * c, rem = tasks % 512;
                const double r = 0.54 * (double)(tasks / 512) + (rem == 0 ? 0.0 : rem <= 256 ? 0.28 : 0.54);
                const double est = r / c + (c > 1 ? 0.03 : 0.0);
                if (est < 0.97 * best) {
                    best = est;
                    sl = c;
                }
            }
        }
        if (sl > 1) {
            p.kslice = (int)((stages + sl - 1) / sl);
            p.slices = (int)((stages + p.kslice - 1) / p.kslice);
        }
    }
    if (p.slices > 1) {
        // one partial tile per slice: tm x t floats
        void *ws = nullptr;
        GFH_TRY(stream_workspace(s, sizeof(float) * (size_t)(p.slices * nblk) * tm * t, &ws));
        p.part = static_cast<float *>(ws);
        GFH_TRY(stream_counters(s, (size_t)nblk, &p.counters));
    }
    const dim3 grid((unsigned)(nblk * p.slices), (unsigned)std::max<int64_t>(d.batch, 1));
    if (t == 256) {
        launch_layouts<256, 256, 2, 4, 2, 1>(d.trans_a, d.trans_b, batched, p, grid, s);
    } else if (t == 128) {
        // One round of tiles (one workgroup per CU): a 3-deep ring (2048^3 NN
        // 143.7 -> 133.7 us); more tiles: 2 stages, two workgroups per CU.
        if (nblk * p.slices * nb <= 256)
            launch_layouts<128, 128, 2, 4, 3, 1>(d.trans_a, d.trans_b, batched, p, grid, s);
        else
            launch_layouts<128, 128, 2, 4, 2, 1>(d.trans_a, d.trans_b, batched, p, grid, s);
    } else if (tm == 32) {
        if (d.trans_b)
            launch_layouts<32, 64, 1, 2, 4, 2>(d.trans_a, true, batched, p, grid, s);
        else
            launch_layouts<32, 64, 1, 2, 2, 2>(d.trans_a, false, batched, p, grid, s);
    } else {
        // Two wave sets splitting each stage's k-groups, so each SIMD runs
        // two waves (1024^3 NN 24.1 -> 22.0 us, 1024 x 1024 x 4096 NN 86.3
        // -> 77.5 us; NT unchanged).  Ring depth: NT 4 stages, NN 2 (of
        // 2 / 3 / 4 / 6: NN 22.0 / 22.8 / 22.2 / 22.4 us at 1024^3).
        if (d.trans_b)
            launch_layouts<64, 64, 2, 2, 4, 2>(d.trans_a, true, batched, p, grid, s);
        else
            launch_layouts<64, 64, 2, 2, 2, 2>(d.trans_a, false, batched, p, grid, s);
    }
    return check_launch("sgemm (direct-to-LDS tiles)");
}

}  // namespace gfh
