// quant_math.hpp -- the reference's int8 quantization arithmetic
// (ghostflow-nn/src/quantization.rs:77-204) as device functions, shared by the
// quantize kernels and the INT8 linear that quantizes its own activations:
//   min/max folds ignore NaN (f32::min / f32::max  ->  fminf / fmaxf);
//   symmetric : scale = max(|min|, |max|) / 127, zp = 0
//   asymmetric: scale = (max - min) / 255, zp = ((-min / scale) - 128).round() as i8
//   q = ((x / scale).round() as i32 + zp).clamp(-128, 127)
// `/` is the correctly rounded IEEE f32 division (hipcc's default), `round`
// is half away from zero, `as` casts saturate with NaN -> 0, and the i32 add
// wraps as in a release build.  No multiply-add here can be contracted.
#pragma once

#include "common.hpp"

namespace gfh {
namespace qmath {

__device__ __forceinline__ int32_t sat_f32_to_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

__device__ __forceinline__ int8_t sat_f32_to_i8(float f) {
    if (f != f) return 0;
    if (f >= 127.0f) return 127;
    if (f <= -128.0f) return -128;
    return (int8_t)(int32_t)f;
}

__device__ __forceinline__ void quant_params(float mn, float mx, bool symmetric, float &scale, int8_t &zp) {
    if (symmetric) {
        const float absmax = fmaxf(fabsf(mn), fabsf(mx));
        scale = absmax / 127.0f;
        zp = 0;
    } else {
        scale = (mx - mn) / 255.0f;
        const float t = (-mn) / scale - 128.0f;
        zp = sat_f32_to_i8(roundf(t));
    }
}

__device__ __forceinline__ int8_t quant_one(float x, float scale, int32_t zp) {
    const uint32_t sum = (uint32_t)sat_f32_to_i32(roundf(x / scale)) + (uint32_t)zp;
    int32_t q = (int32_t)sum;
    q = q < -128 ? -128 : (q > 127 ? 127 : q);
    return (int8_t)q;
}

__device__ __forceinline__ uint32_t quant4(f32x4 v, float scale, int32_t zp) {
    // (vector elements are copied to scalars first: this compiler bit-casts
    // an element lvalue from the vector start)
    const float v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
    const uint32_t b0 = (uint8_t)quant_one(v0, scale, zp);
    const uint32_t b1 = (uint8_t)quant_one(v1, scale, zp);
    const uint32_t b2 = (uint8_t)quant_one(v2, scale, zp);
    const uint32_t b3 = (uint8_t)quant_one(v3, scale, zp);
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// Workgroup-wide (min, max) of NT threads: wave shuffles, then LDS across
// waves.  Every thread of the workgroup must call it.
template <int NT>
__device__ __forceinline__ void block_minmax(float &mn, float &mx) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, off));
        mx = fmaxf(mx, __shfl_xor(mx, off));
    }
    __shared__ float smn[NT / 64], smx[NT / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        smn[wave] = mn;
        smx[wave] = mx;
    }
    __syncthreads();
    mn = smn[0];
    mx = smx[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) {
        mn = fminf(mn, smn[w]);
        mx = fmaxf(mx, smx[w]);
    }
    __syncthreads();
}

}  // namespace qmath
}  // namespace gfh
