// sgemm.hip -- fp32 GEMM on CDNA4 f32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Computes C = alpha * op(A) . op(B) + beta * C (+ bias[n]) for row-major
// operands, the work of Tensor::matmul / matmul_blocked
// (ghostflow-core/src/ops/matmul.rs:91-119), batched_matmul (:122-170) and
// Linear::forward (ghostflow-nn/src/linear.rs:56-69).
//
// Design (one 256-thread workgroup = 4 wave64s per BM x BN output tile):
//  * Each wave owns a WM x WN sub-tile held as (WM/32) x (WN/32) 32x32 MFMA
//    accumulators (16 f32 per lane each).
//  * K advances in BK-wide stages.  Global -> register loads for stage t+1
//    are issued before the MFMAs of stage t, then stored into the other LDS
//    buffer: two LDS buffers, one barrier per stage.
//  * LDS tiles keep the global layout of each operand (no transposing
//    stores): a K-contiguous operand (A, or B given as [n,k]) is read as one
//    16-byte ds_read per 4 k-steps; an M/N-contiguous operand (B given as
//    [k,n], or A given as [k,m]) is read as 4 scalar ds_reads, conflict-free
//    across the 32 lanes that share a k.  Row strides are padded by 4 floats.
//  * Within a group of 8 k values, lanes 0-31 supply k0..k0+3 and lanes
//    32-63 supply k0+4..k0+7 to the 4 consecutive MFMAs (the k <-> MFMA-step
//    assignment is the same for both operands, so the products pair up).
//  * Workgroups are renumbered so that consecutive tiles land on the same
//    XCD (the dispatcher deals workgroups round-robin over the 8 XCDs), and
//    tiles are walked in GROUP_M-row bands so concurrently running tiles
//    share A row panels and B column panels in that XCD's L2.
#include "common.hpp"
#include "kernels.hpp"

// Every multiply and add below is its own f32 rounding, as in the reference
// (rustc never contracts a*b+c into an FMA); the MFMA accumulation itself is
// not affected by this pragma.
#pragma clang fp contract(off)

namespace gfh {
namespace {

constexpr int kThreads = 256;
constexpr int kPad = 4;
constexpr int kGroupM = 8;

struct SgemmParams {
    const float *a;
    const float *b;
    float *c;
    const float *bias;
    int64_t m, n, k;
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;
    int64_t batch_a, batch_b;
    float alpha, beta;
    int tiles_m, tiles_n;
};

// Tile geometry in LDS.  K-contiguous: [rows][BK + pad];  MN-contiguous:
// [BK][rows + pad].
template <int ROWS, int BK, bool KCONTIG>
struct LdsTile {
    static constexpr int kStride = KCONTIG ? (BK + kPad) : (ROWS + kPad);
    static constexpr int kFloats = KCONTIG ? ROWS * kStride : BK * kStride;
};

// Loads one ROWS x BK stage of an operand into registers.  `kcontig`
// operands are stored [rows][ld] with k fastest; the others [k][ld] with rows
// fastest.  Out-of-range elements read as 0.
template <int ROWS, int BK, bool KCONTIG, bool VEC>
struct StageLoader {
    static constexpr int kVecs = ROWS * BK / 4;
    static constexpr int kPerThread = kVecs / kThreads;
    static_assert(kVecs % kThreads == 0, "tile must split evenly over the workgroup");
    f32x4 r[kPerThread];

    __device__ __forceinline__ void load(const float *__restrict__ base, int64_t ld, int64_t row0,
                                         int64_t rows_total, int64_t k0, int64_t k_total, int tid) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = tid + i * kThreads;
            int64_t row, kk;
            if (KCONTIG) {
                row = row0 + idx / (BK / 4);
                kk = k0 + (idx % (BK / 4)) * 4;
            } else {
                kk = k0 + idx / (ROWS / 4);
                row = row0 + (idx % (ROWS / 4)) * 4;
            }
            // (outer, inner) coordinates in the operand's storage order.
            const int64_t outer = KCONTIG ? row : kk;
            const int64_t inner = KCONTIG ? kk : row;
            const int64_t outer_n = KCONTIG ? rows_total : k_total;
            const int64_t inner_n = KCONTIG ? k_total : rows_total;
            const float *p = base + outer * ld + inner;
            if (VEC && outer < outer_n && inner + 3 < inner_n) {
                r[i] = *reinterpret_cast<const f32x4 *>(p);
            } else {
                f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (outer < outer_n) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (inner + e < inner_n) v[e] = p[e];
                }
                r[i] = v;
            }
        }
    }

    __device__ __forceinline__ void store(float *lds, int tid) const {
        using T = LdsTile<ROWS, BK, KCONTIG>;
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = tid + i * kThreads;
            int o, in;
            if (KCONTIG) {
                o = idx / (BK / 4);
                in = (idx % (BK / 4)) * 4;
            } else {
                o = idx / (ROWS / 4);
                in = (idx % (ROWS / 4)) * 4;
            }
            *reinterpret_cast<f32x4 *>(lds + o * T::kStride + in) = r[i];
        }
    }
};

// Fragment of 32 rows x 8 k (one k-group) for 4 MFMA steps.
template <int ROWS, int BK, bool KCONTIG>
__device__ __forceinline__ f32x4 load_frag(const float *lds, int row0, int kg, int lane) {
    using T = LdsTile<ROWS, BK, KCONTIG>;
    const int r = row0 + (lane & 31);
    const int kb = kg * 8 + 4 * (lane >> 5);
    if (KCONTIG) {
        return *reinterpret_cast<const f32x4 *>(lds + r * T::kStride + kb);
    } else {
        f32x4 v;
#pragma unroll
        for (int s = 0; s < 4; ++s) v[s] = lds[(kb + s) * T::kStride + r];
        return v;
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(kThreads) void sgemm_mfma_kernel(SgemmParams p) {
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int WAVES_N = BN / WN;
    static_assert((BM / WM) * (BN / WN) == kThreads / 64, "4 waves per workgroup");
    constexpr bool A_KC = !TA;  // A [m,k] is k-contiguous
    constexpr bool B_KC = TB;   // B given as [n,k] is k-contiguous
    using TileA = LdsTile<BM, BK, A_KC>;
    using TileB = LdsTile<BN, BK, B_KC>;

    __shared__ __attribute__((aligned(16))) float lds[2 * (TileA::kFloats + TileB::kFloats)];
    float *const lds_a0 = lds;                          // two A buffers, then two B buffers
    float *const lds_b0 = lds + 2 * TileA::kFloats;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave / WAVES_N) * WM;
    const int wn0 = (wave % WAVES_N) * WN;

    // Workgroup -> tile: XCD-contiguous renumbering, then GROUP_M bands.
    const int nblk = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int group_size = kGroupM * p.tiles_n;
    const int group = bid / group_size;
    const int first_m = group * kGroupM;
    const int gm = min(p.tiles_m - first_m, kGroupM);
    const int in_group = bid - group * group_size;
    const int tile_m = first_m + in_group % gm;
    const int tile_n = in_group / gm;
    const int64_t m0 = (int64_t)tile_m * BM;
    const int64_t n0 = (int64_t)tile_n * BN;

    const int64_t batch = blockIdx.z;
    const float *A = p.a + (batch % p.batch_a) * p.stride_a;
    const float *B = p.b + (batch % p.batch_b) * p.stride_b;
    float *Cm = p.c + batch * p.stride_c;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    StageLoader<BM, BK, A_KC, VEC> ga;
    StageLoader<BN, BK, B_KC, VEC> gb;
    const int64_t nstages = (p.k + BK - 1) / BK;

    if (nstages > 0) {
        ga.load(A, p.lda, m0, p.m, 0, p.k, tid);
        gb.load(B, p.ldb, n0, p.n, 0, p.k, tid);
        ga.store(lds_a0, tid);
        gb.store(lds_b0, tid);
    }
    __syncthreads();

    for (int64_t st = 0; st < nstages; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nstages;
        if (more) {
            ga.load(A, p.lda, m0, p.m, (st + 1) * BK, p.k, tid);
            gb.load(B, p.ldb, n0, p.n, (st + 1) * BK, p.k, tid);
        }
        const float *la = lds_a0 + cur * TileA::kFloats;
        const float *lb = lds_b0 + cur * TileB::kFloats;
#pragma unroll
        for (int kg = 0; kg < BK / 8; ++kg) {
            f32x4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = load_frag<BM, BK, A_KC>(la, wm0 + i * 32, kg, lane);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[j] = load_frag<BN, BK, B_KC>(lb, wn0 + j * 32, kg, lane);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
        }
        if (more) {
            ga.store(lds_a0 + (cur ^ 1) * TileA::kFloats, tid);
            gb.store(lds_b0 + (cur ^ 1) * TileB::kFloats, tid);
        }
        __syncthreads();
    }

    // Epilogue: 32x32 accumulator layout -- lane l, register r holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t col = n0 + wn0 + j * 32 + (lane & 31);
            if (col >= p.n) continue;
            const float bv = p.bias ? p.bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= p.m) continue;
                float v = p.alpha * acc[i][j][r];
                float *dst = Cm + row * p.ldc + col;
                if (p.beta != 0.f) v = v + p.beta * *dst;
                if (p.bias) v = v + bv;
                *dst = v;
            }
        }
}

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VEC>
int launch_tiles(const SgemmParams &p0, int64_t batch, hipStream_t s) {
    SgemmParams p = p0;
    p.tiles_m = (int)((p.m + BM - 1) / BM);
    p.tiles_n = (int)((p.n + BN - 1) / BN);
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
    hipLaunchKernelGGL((sgemm_mfma_kernel<BM, BN, BK, WM, WN, TA, TB, VEC>), grid, dim3(kThreads), 0, s, p);
    return check_launch("sgemm");
}

// Tile size by problem size: 128 x 128 tiles (64 x 64 per wave) give the
// most MFMA work per LDS byte, but a launch needs hundreds of workgroups to
// keep all 1024 SIMDs busy.  Measured (square, NN): 1024^3 88.7 us at
// 128x128 (64 workgroups), 50.4 at 128x64, 30.9 at 64x64 with BK = 64;
// 2048^3 170 / 159 / 173 us; 4096^3 1104 / 1221 / 1318 us.
template <bool TA, bool TB, bool VEC>
int launch_variant(const SgemmParams &p, int64_t batch, hipStream_t s) {
    const int64_t t128 = ((p.m + 127) / 128) * ((p.n + 127) / 128) * batch;
    if (t128 >= 512) return launch_tiles<128, 128, 32, 64, 64, TA, TB, VEC>(p, batch, s);
    if (t128 >= 128) return launch_tiles<128, 64, 32, 64, 32, TA, TB, VEC>(p, batch, s);
    return launch_tiles<64, 64, 64, 32, 32, TA, TB, VEC>(p, batch, s);
}

}  // namespace

bool sgemm_nt_group_fits(const SgemmDesc *d, int count) {
    return gemv_nt_group_fits(d, count) || gemm_nt_skinny_group_fits(d, count);
}

int launch_sgemm_nt_group(const SgemmDesc *d, int count, hipStream_t s) {
    if (gemv_nt_group_fits(d, count)) return launch_gemv_nt_group(d, count, s);
    if (gemm_nt_skinny_group_fits(d, count)) return launch_gemm_nt_skinny_group(d, count, s);
    return set_error(GFH_INVALID_SHAPE, "sgemm: these products do not share one launch");
}

// Tensor::matmul at decode batch sizes, x [m, k] . W [k, n] with m <= 16 and
// packed rows: the decode GEMV (gemv.hip) streams W once per 8 rows of x,
// with the same epilogue.  (W [4096, 14336]: 38-39 us at m = 1-8, where the
// tile kernels took 106 us.)
namespace {
bool gemv_nn_fits(const SgemmDesc &d) {
    return !d.trans_a && !d.trans_b && d.batch <= 1 && d.batch_a <= 1 && d.batch_b <= 1 && d.m >= 1 && d.m <= 16 &&
           d.k > 0 && d.n > 0 && d.lda == d.k && d.ldb == d.n && d.ldc == d.n;
}
}  // namespace

int launch_sgemm(const SgemmDesc &d, hipStream_t s) {
    // x . W^T with at most 8 rows of x: a tile of this kernel would leave
    // most of its MFMA rows empty and its grid far too small to stream W.
    if (gemv_nt_fits(d)) return launch_gemv_nt(d, s);
    if (gemv_nn_fits(d)) return launch_gemv_f32_epi(d.a, d.b, d.c, d.m, d.k, d.n, d.alpha, d.beta, d.bias, s);
    // up to 64 rows: the weight streamed straight into f32 MFMA operands
    if (gemm_nt_skinny_fits(d)) return launch_gemm_nt_skinny(d, s);
    // NT / NN on 256 x 256 tiles fed by direct-to-LDS loads, when they fill the GPU
    if (sgemm_big_fits(d)) return launch_sgemm_big(d, s);
    SgemmParams p{};
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
    p.batch_a = d.batch_a;
    p.batch_b = d.batch_b;
    p.alpha = d.alpha;
    p.beta = d.beta;
    // 16-byte vector loads need 16-byte aligned rows and slices.
    const bool vec = aligned16(d.a) && aligned16(d.b) && (d.lda % 4 == 0) && (d.ldb % 4 == 0) &&
                     (d.batch_a <= 1 || d.stride_a % 4 == 0) && (d.batch_b <= 1 || d.stride_b % 4 == 0);
    const int key = (d.trans_a ? 4 : 0) | (d.trans_b ? 2 : 0) | (vec ? 1 : 0);
    switch (key) {
        case 0: return launch_variant<false, false, false>(p, d.batch, s);
        case 1: return launch_variant<false, false, true>(p, d.batch, s);
        case 2: return launch_variant<false, true, false>(p, d.batch, s);
        case 3: return launch_variant<false, true, true>(p, d.batch, s);
        case 4: return launch_variant<true, false, false>(p, d.batch, s);
        case 5: return launch_variant<true, false, true>(p, d.batch, s);
        case 6: return launch_variant<true, true, false>(p, d.batch, s);
        default: return launch_variant<true, true, true>(p, d.batch, s);
    }
}

}  // namespace gfh
