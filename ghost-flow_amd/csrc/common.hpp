// common.hpp -- shared host/device helpers of the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "ghostflow_hip.h"

namespace gfh {

// ---- error reporting (thread-local last error) ---------------------------
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// hipGetLastError after a launch -> GFH_COMPUTATION_FAILED with its text.
int check_launch(const char *what);
// Lazily initializes the device table; returns GFH_SUCCESS or an error code.
int ensure_init();

// ---- argument validation --------------------------------------------------
// Device-pointer check (hipPointerGetAttributes) when pointer checks are on;
// `p` must be non-null.
int check_device_ptr(const void *p, const char *name);
// Null check + device check for a required pointer.
int require_ptr(const void *p, const char *name);
// Required pointer to `bytes` bytes of device memory: non-null (unless
// bytes == 0), and, with pointer checks on, [p, p + bytes) inside one device
// allocation (hipMemGetAddressRange), so an undersized or host buffer is an
// error instead of a GPU memory fault.
int require_range(const void *p, size_t bytes, const char *name);
// Same for a nullable pointer: NULL is accepted.
int optional_range(const void *p, size_t bytes, const char *name);
int set_pointer_checks(int enabled);
const char *last_error();
// 16-byte alignment helper.
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- stream-ordered scratch ----------------------------------------------
// Uses the caller's workspace when given (and large enough), otherwise
// hipMallocAsync on the stream; releases with hipFreeAsync on destruction.
class Scratch {
  public:
    Scratch() = default;
    ~Scratch();
    int acquire(void *user, size_t user_bytes, size_t need, hipStream_t s);
    void *ptr() const { return p_; }

  private:
    void *p_ = nullptr;
    bool owned_ = false;
    hipStream_t s_ = nullptr;
};

inline hipStream_t as_stream(gfh_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Per (device, stream) device state owned by the library, reused by every
// call on that stream (calls on one stream are serialized by the stream, so
// they can share it; other streams get their own):
//  * int32 counters that are all zero whenever no kernel of the stream is
//    running -- a kernel that counts arrivals in them must leave every
//    counter it used at 0;
//  * a scratch buffer for partial results.
// Both are allocated (and the counters zeroed) stream-ordered on first use,
// grow on demand, and are released at shutdown.
int stream_counters(hipStream_t s, size_t count, int **out);
int stream_workspace(hipStream_t s, size_t bytes, void **out);
void release_stream_state();

// Compute units of the current device (queried once per device).
int device_cu_count();

// Workgroup w of a launch runs on XCD w % 8 (round-robin dispatch over the
// 8 XCDs, each with its own L2).  This renumbering gives every XCD one
// contiguous range of tile ids -- XCD x takes q + (x < r) of them from
// x q + min(x, r), q = n / 8, r = n % 8 -- so tiles that share operand rows
// (neighbours in tile order) share an L2.  A bijection on [0, n) for any n.
__device__ __forceinline__ int xcd_chunked(int w, int n) {
    const int q = n >> 3, r = n & 7, x = w & 7;
    return x * q + (x < r ? x : r) + (w >> 3);
}

// ---- split-K arrival protocol ------------------------------------------------
// Kernels that split K over workgroups (the decode GEMVs, the skinny int8 and
// fp32 linears, KV-cache attention) combine their partials in the same
// launch:
//   1. each workgroup (or wave) stores its partial with agent-scope relaxed
//      atomic stores; these bypass the per-XCD L2 (which is not coherent
//      across XCDs) and complete at the device coherence point;
//   2. s_waitcnt vmcnt(0): the storing thread waits until its stores are
//      acknowledged; an __atomic_signal_fence before it keeps the compiler
//      from moving a store past the wait;
//   3. after a barrier (when several threads stored), one thread counts the
//      arrival with an agent-scope relaxed fetch_add; the one that reads
//      slices - 1 is the last to arrive;
//   4. the last arriver loads the other partials with agent-scope relaxed
//      loads (also served by the coherence point), sums them in a fixed order
//      and returns the counter to 0.
// Ordering relied on: a partial store acknowledged before the arrival is
// counted is visible to an agent-scope load that the last arriver issues
// after reading the count.  This is the vmcnt form of release / acquire: the
// HIP memory model's release / acquire fences order the same accesses but
// compile to a whole-L2 writeback / invalidate on this target (measured: the
// int8 GEMV fell to 1.8 TB/s).  It would break if a store were moved past
// the wait (the signal fences prevent that in the compiler) or if hardware
// acknowledged an agent-scope store before it reached the coherence point.

}  // namespace gfh

// Propagate a non-zero status.
#define GFH_TRY(expr)                  \
    do {                               \
        int gfh_rc__ = (expr);         \
        if (gfh_rc__ != GFH_SUCCESS) { \
            return gfh_rc__;           \
        }                              \
    } while (0)

// ---- device-side vector types and MFMA wrappers --------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Cache-policy operand of __builtin_amdgcn_global_load_lds that sets the
// instruction's nt bit (gfx950: global_load_lds_dwordx4 ... nt), the hint
// __builtin_nontemporal_load gives an ordinary load: for streams read once,
// such as a weight whose every byte one workgroup consumes.
constexpr int kNtHint = 2;

// 16-byte partial-result traffic of the split-K protocol below: raw buffer
// loads and stores with the sc1 cache bit, the bit an agent-scope relaxed
// atomic load or store carries (global_load_dword / global_store_dword ...
// sc1), so they complete at the device coherence point like those, four
// dwords per instruction instead of one.  The buffer resource bounds every
// access to `bytes` (the gfx9 raw-buffer word 3: 32-bit data format); `bytes`
// must fit 32 bits.
constexpr int kScDevice = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_buffer(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// ---- cross-lane sums without LDS round trips ---------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float readlane_f(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
// Sum over each row of 16 lanes, in every lane of the row: quad xor 1 and
// xor 2 (DPP quad_perm), then rotations by 4 and 8 within the row.  Lanes of
// a row may differ in the last bit (the rotations associate differently).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x124>(v);  // row_ror:4
    v += dpp_mov<0x128>(v);  // row_ror:8
    return v;
}
// Sum over the 64 lanes, bit-identical in every lane (row totals read out
// with readlane and added in a fixed order).  A __shfl_xor ladder would be
// six dependent ds_bpermute round trips.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}
// Sum over each half-wave (lanes 0-31, 32-63), bit-identical across it.
__device__ __forceinline__ float half_wave_sum(float v) {
    v = row16_sum(v);
    const float lo = readlane_f(v, 0) + readlane_f(v, 16);
    const float hi = readlane_f(v, 32) + readlane_f(v, 48);
    return (threadIdx.x & 32) ? hi : lo;
}

// ---- four lanes c, c + 16, c + 32, c + 48 -----------------------------------
//
// In the 16x16x4 MFMA layouts (lane l holds column l % 16 in quarter l / 16)
// a column's values sit in lanes c, c + 16, c + 32, c + 48.  These fold them
// with gfx950's lane swaps: v_permlane16_swap pairs lane l with l ^ 16 and
// v_permlane32_swap pairs it with l ^ 32 (both halves of each result hold
// the two values), VALU ops instead of LDS-path permutes.  Every lane of the
// four ends with the same result.
__device__ __forceinline__ float quarter_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quarter_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// The partner's copy of x across lane bit 4 (l ^ 16) or bit 5 (l ^ 32).
template <int BIT>
__device__ __forceinline__ unsigned swap_partner(unsigned x, int lane) {
    const auto a = BIT == 4 ? __builtin_amdgcn_permlane16_swap(x, x, false, false)
                            : __builtin_amdgcn_permlane32_swap(x, x, false, false);
    // a holds {lower lane's value, upper lane's value} of the pair
    return ((lane >> BIT) & 1) ? a[0] : a[1];
}
// fp64 sum over the four lanes, in a fixed order for every lane:
// (quarter 0 + quarter 1) + (quarter 2 + quarter 3).
__device__ __forceinline__ double quarter_sum_f64(double x, int lane) {
    auto partner = [&](double v, auto bit) {
        constexpr int B = decltype(bit)::value;
        const unsigned long long u = __double_as_longlong(v);
        const unsigned lo = swap_partner<B>((unsigned)u, lane), hi = swap_partner<B>((unsigned)(u >> 32), lane);
        return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
    };
    const double y = partner(x, std::integral_constant<int, 4>{});
    x = ((lane >> 4) & 1) ? y + x : x + y;
    const double z = partner(x, std::integral_constant<int, 5>{});
    return ((lane >> 5) & 1) ? z + x : x + z;
}
// The largest value over the four lanes and its key; ties go to
// the smaller key, so every lane picks the same one.
__device__ __forceinline__ void quarter_argmax(float &v, int &key, int lane) {
    auto pick = [&](auto bit) {
        constexpr int B = decltype(bit)::value;
        const float pv = __uint_as_float(swap_partner<B>(__float_as_uint(v), lane));
        const int pk = (int)swap_partner<B>((unsigned)key, lane);
        if (pv > v || (pv == v && pk < key)) {
            v = pv;
            key = pk;
        }
    };
    pick(std::integral_constant<int, 4>{});
    pick(std::integral_constant<int, 5>{});
}

// silu(g) * up as the reference computes it (activation.rs:117-122 and
// arithmetic.rs:39-45): negate, expf, add, IEEE division, multiply -- each
// a separate f32 rounding.
__device__ __forceinline__ float silu_mul1(float g, float u) {
#pragma clang fp contract(off)
    const float s = g / (1.0f + expf(-g));
    return s * u;
}

// (min, max) over the 64 lanes, NaN-ignoring like f32::min / f32::max.
__device__ __forceinline__ void wave_minmax(float &mn, float &mx) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, off));
        mx = fmaxf(mx, __shfl_xor(mx, off));
    }
}
