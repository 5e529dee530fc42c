// attn_tiles.hpp -- pieces shared by the tiled attention kernels
// (attention.hip, flash_attention.hip): 32-key K/V tiles staged through
// registers into padded LDS rows, and the key each score accumulator
// register holds.
#pragma once

#include "common.hpp"

namespace gfh {
namespace attn {

constexpr int kBKV = 32;  // keys per LDS tile

// S^T = K . Q^T on v_mfma_f32_32x32x2_f32: lane (c = l % 32, h = l / 32),
// accumulator register r holds key 8 (r / 4) + 4 h + r % 4 of the tile for
// query c.
__device__ __forceinline__ int key_of(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// One 32-key x DMAX tile of K or V staged through registers: DMAX * 8
// float4 per tile spread over NT threads; LDS rows padded to DMAX + 4 floats.
// Keys past nkeys and dims past d load as zero (d % 4 == 0, rows 16-byte
// aligned).
template <int DMAX, int NT>
struct KvStage {
    static constexpr int kPer = kBKV * DMAX / 4 / NT;
    static constexpr int kStride = DMAX + 4;
    f32x4 r[kPer];

    __device__ __forceinline__ void load(const float *__restrict__ base, int64_t key0, int64_t nkeys, int64_t d,
                                         int64_t rs, int tid) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int idx = tid + i * NT;
            const int key = idx / (DMAX / 4);
            const int dim = (idx % (DMAX / 4)) * 4;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (key0 + key < nkeys && dim < d) v = *reinterpret_cast<const f32x4 *>(base + (key0 + key) * rs + dim);
            r[i] = v;
        }
    }
    __device__ __forceinline__ void store(float *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int idx = tid + i * NT;
            const int key = idx / (DMAX / 4);
            const int dim = (idx % (DMAX / 4)) * 4;
            *reinterpret_cast<f32x4 *>(lds + key * kStride + dim) = r[i];
        }
    }
};

}  // namespace attn
}  // namespace gfh
