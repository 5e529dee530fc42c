// attn_tiles.hpp -- pieces shared by the tiled attention kernels
// (attention.hip, flash_attention.hip): 32-key K/V tiles staged through
// registers into padded LDS rows, and the key each score accumulator
// register holds.
#pragma once

#include <type_traits>

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

// ---- direct-to-LDS tiles -------------------------------------------------------
//
// A 32-key x DMAX tile (DMAX = 64 or 128) requested straight into LDS with
// global_load_lds_dwordx4: no staging registers, no LDS store instructions.
// One load instruction fills 1 KB of LDS; which global 16-byte chunk lands
// in which LDS slot is free per lane, so each operand gets the layout its
// reads want:
//  * K tiles are chunk-major: chunk q of key r at slot q * 32 + r.  A score
//    fragment read (ds_read_b128; 16 lanes on keys 0..15 at one chunk) is
//    256 contiguous bytes, and the address is a lane base plus a constant
//    per chunk.  Instruction i loads chunks 2i, 2i + 1 of all 32 keys.
//  * V tiles are key-major, chunk q of key r at chunk q ^ (4 * bits 2-3 of
//    r): a P.V operand read of the 16x16x4 layouts (four lane quarters on
//    keys 4 apart, 16 consecutive dims each) then falls on four disjoint
//    16-bank groups.  Instruction i loads 1024 / (4 DMAX) whole keys.
// Keys past nkeys read the last key and chunks past d read chunk 0 of the
// row: finite values that meet a -inf score (weight 0) or a zero query dim.
typedef __attribute__((address_space(3))) void *lds_ptr_t;
typedef __attribute__((address_space(1))) void *glb_ptr_t;

template <int DMAX, int NT, bool IS_V>
struct KvLds {
    static_assert(DMAX == 64 || DMAX == 128, "direct-to-LDS tiles cover 64 or 128 dims");
    static constexpr int kTileFloats = kBKV * DMAX;
    static constexpr int kInstr = kTileFloats * 4 / 1024;  // load instructions per tile
    static constexpr int kPerWave = kInstr / (NT / 64);
    static_assert(kPerWave >= 1 && kPerWave * (NT / 64) == kInstr, "whole instructions per wave");
    static constexpr int kChunks = DMAX / 4;  // 16-byte chunks per key

    // This wave's share of the requests for keys key0 .. key0 + 31 (row
    // stride rs floats, 16-byte aligned rows, d % 4 == 0, nkeys >= 1).
    __device__ __forceinline__ static void issue(const float *__restrict__ base, int64_t key0, int64_t nkeys,
                                                 int64_t d, int64_t rs, float *lds, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < kPerWave; ++i) {
            const int ins = wave * kPerWave + i;
            int row, lc;
            if (IS_V) {
                row = ins * (64 / kChunks) + lane / kChunks;
                lc = (lane % kChunks) ^ (4 * ((row >> 2) & 3));
            } else {
                row = lane & 31;
                lc = 2 * ins + (lane >> 5);
            }
            if (4 * lc >= d) lc = 0;
            const int64_t key = min(key0 + row, nkeys - 1);
            __builtin_amdgcn_global_load_lds((glb_ptr_t)(base + key * rs + 4 * lc), (lds_ptr_t)(lds + ins * 256), 16,
                                             0, 0);
        }
    }
};

// s_waitcnt vmcnt(0): this wave's global loads (and LDS-bound requests) are done.
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

}  // namespace attn
}  // namespace gfh
