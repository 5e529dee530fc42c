// tensor_api.hip -- GhostFlow's Tensor-level C API (ghostflow.h) over HBM
// tensors: the entry points of ghostflow-ffi/src/lib.rs:60-337 with the
// same argument checks, error codes and ownership, each tensor an fp32
// buffer on the device that was current at its creation.
//
//  * create / data: one host <-> device copy each; zeros / ones: a fill
//    kernel.
//  * add / mul: one element-wise kernel over the broadcast shape of
//    Shape::broadcast_with (ghostflow-core/src/shape.rs:49-80); operand
//    element offsets follow compute_broadcast_strides / _index
//    (ghostflow-core/src/ops/arithmetic.rs:180-215): stride 0 on a stretched
//    dimension.  Dimensions are merged where both operands stay contiguous
//    across them, so the common shapes (same shape, bias rows, scalars) run
//    with one or two index divisions per element.
//  * matmul: gfh_sgemm (2-D) or gfh_sgemm_strided_batched with the
//    reference's batch indexing (ghostflow-core/src/ops/matmul.rs:122-170).
//  * reshape: a new handle on the same buffer (shared ownership).
// Everything runs on the device's default stream in call order.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <new>
#include <vector>

#include "common.hpp"
#include "ghostflow.h"

#pragma clang fp contract(off)

namespace {

struct DeviceBuffer {
    float *p = nullptr;
    int device = 0;
    ~DeviceBuffer() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace

// The opaque handle of ghostflow.h.
struct GhostFlowTensor {
    std::vector<size_t> dims;
    size_t numel = 1;
    std::shared_ptr<DeviceBuffer> buf;  // numel floats (null when numel == 0)
};

namespace {

using gfh::set_error;

constexpr int kMaxDims = 16;  // after merging; more is refused with ComputationFailed
constexpr int kThreads = 256;

GhostFlowError as_ffi(int status) {
    switch (status) {
        case GFH_SUCCESS: return Success;
        case GFH_INVALID_SHAPE: return InvalidShape;
        case GFH_INVALID_DATA: return InvalidData;
        case GFH_NULL_POINTER: return NullPointer;
        case GFH_ALLOCATION_FAILED: return AllocationFailed;
        case GFH_COMPUTATION_FAILED: return ComputationFailed;
        default: return Unknown;
    }
}

// Element count of a shape, false on size_t overflow.  An empty shape is a
// scalar (one element), as Shape::numel's empty product.
bool shape_numel(const uintptr_t *shape, uintptr_t len, size_t *out) {
    size_t n = 1;
    for (uintptr_t i = 0; i < len; ++i) {
        if (shape[i] != 0 && n > SIZE_MAX / shape[i]) return false;
        n *= shape[i];
    }
    *out = n;
    return true;
}

// Restores the caller's current device on scope exit.
class DeviceScope {
  public:
    explicit DeviceScope(int dev) {
        ok_ = hipGetDevice(&prev_) == hipSuccess;
        if (ok_ && prev_ != dev) ok_ = hipSetDevice(dev) == hipSuccess, switched_ = ok_;
    }
    ~DeviceScope() {
        if (switched_) (void)hipSetDevice(prev_);
    }
    bool ok() const { return ok_; }

  private:
    int prev_ = 0;
    bool ok_ = false, switched_ = false;
};

// A new tensor of the given dims on the current device, uninitialized.
int new_tensor(const std::vector<size_t> &dims, GhostFlowTensor **out) {
    std::unique_ptr<GhostFlowTensor> t(new GhostFlowTensor);
    t->dims = dims;
    t->numel = 1;
    for (size_t d : dims) {
        if (d != 0 && t->numel > SIZE_MAX / 4 / d) return set_error(GFH_INVALID_SHAPE, "tensor of too many elements");
        t->numel *= d;
    }
    t->buf = std::make_shared<DeviceBuffer>();
    GFH_TRY(gfh::ensure_init());
    if (hipGetDevice(&t->buf->device) != hipSuccess) return set_error(GFH_COMPUTATION_FAILED, "no current device");
    if (t->numel > 0) {
        const hipError_t e = hipMalloc(&t->buf->p, t->numel * sizeof(float));
        if (e != hipSuccess) {
            (void)hipGetLastError();
            t->buf->p = nullptr;
            return set_error(GFH_ALLOCATION_FAILED, "hipMalloc of %zu bytes: %s", t->numel * sizeof(float),
                             hipGetErrorString(e));
        }
    }
    *out = t.release();
    return GFH_SUCCESS;
}

__global__ void fill_kernel(float *p, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

unsigned grid_for(size_t n) {
    const size_t g = (n + kThreads - 1) / kThreads;
    return (unsigned)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

// Broadcast layout of c = op(a, b) after merging: nd dims (outermost
// first) with the operands' element strides (0 where stretched).
struct Bcast {
    int nd;
    int64_t dim[kMaxDims];
    int64_t sa[kMaxDims], sb[kMaxDims];
};

template <int OP>
__device__ __forceinline__ float apply(float x, float y) {
    if constexpr (OP == 0)
        return x + y;
    else
        return x * y;
}

// Same shape: c[i] = op(a[i], b[i]), 16-byte accesses when all three are
// aligned (the last n % 4 elements then by the first threads).
template <int OP>
__global__ void binary_same_kernel(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ c,
                                   size_t n, int vec) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const size_t n4 = n / 4;
        for (size_t j = gid; j < n4; j += stride) {
            const float4 x = reinterpret_cast<const float4 *>(a)[j], y = reinterpret_cast<const float4 *>(b)[j];
            reinterpret_cast<float4 *>(c)[j] =
                make_float4(apply<OP>(x.x, y.x), apply<OP>(x.y, y.y), apply<OP>(x.z, y.z), apply<OP>(x.w, y.w));
        }
        const size_t t = n4 * 4 + gid;
        if (t < n) c[t] = apply<OP>(a[t], b[t]);
        return;
    }
    for (size_t i = gid; i < n; i += stride) c[i] = apply<OP>(a[i], b[i]);
}

// General broadcast: flat index i of c decomposed innermost-first over the
// merged dims, as compute_broadcast_index (arithmetic.rs:204-215).
template <int OP>
__global__ void binary_bcast_kernel(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ c,
                                    size_t n, Bcast d) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        size_t rem = i;
        int64_t ia = 0, ib = 0;
        for (int k = d.nd - 1; k >= 0; --k) {
            const int64_t coord = (int64_t)(rem % (size_t)d.dim[k]);
            rem /= (size_t)d.dim[k];
            ia += coord * d.sa[k];
            ib += coord * d.sb[k];
        }
        c[i] = apply<OP>(a[ia], b[ib]);
    }
}

// Shape::broadcast_with: trailing alignment, equal or one of them 1.
bool broadcast_dims(const std::vector<size_t> &a, const std::vector<size_t> &b, std::vector<size_t> *out) {
    const size_t nd = a.size() > b.size() ? a.size() : b.size();
    out->assign(nd, 0);
    for (size_t i = 0; i < nd; ++i) {
        const size_t x = i < a.size() ? a[a.size() - 1 - i] : 1;
        const size_t y = i < b.size() ? b[b.size() - 1 - i] : 1;
        if (x == y || y == 1)
            (*out)[nd - 1 - i] = x;
        else if (x == 1)
            (*out)[nd - 1 - i] = y;
        else
            return false;
    }
    return true;
}

// compute_broadcast_strides (arithmetic.rs:180-201) of `shape` against the
// result dims.
std::vector<int64_t> bcast_strides(const std::vector<size_t> &shape, const std::vector<size_t> &target) {
    const size_t nd = target.size(), off = nd - shape.size();
    std::vector<int64_t> st(nd, 0);
    int64_t stride = 1;
    for (size_t i = shape.size(); i-- > 0;) {
        if (shape[i] == target[i + off]) {
            st[i + off] = stride;
            stride *= (int64_t)shape[i];
        }
    }
    return st;
}

template <int OP>
int binary(const GhostFlowTensor *a, const GhostFlowTensor *b, GhostFlowTensor **out, const char *name) {
    if (!a || !b || !out) return set_error(GFH_NULL_POINTER, "%s: null argument", name);
    if (a->buf->device != b->buf->device)
        return set_error(GFH_COMPUTATION_FAILED, "%s: operands on devices %d and %d", name, a->buf->device,
                         b->buf->device);
    std::vector<size_t> dims;
    if (!broadcast_dims(a->dims, b->dims, &dims))
        return set_error(GFH_COMPUTATION_FAILED, "%s: shapes do not broadcast", name);
    DeviceScope scope(a->buf->device);
    if (!scope.ok()) return set_error(GFH_COMPUTATION_FAILED, "%s: cannot select device %d", name, a->buf->device);
    GhostFlowTensor *c = nullptr;
    GFH_TRY(new_tensor(dims, &c));
    std::unique_ptr<GhostFlowTensor> guard(c);
    if (c->numel > 0) {
        const float *pa = a->buf->p, *pb = b->buf->p;
        float *pc = c->buf->p;
        if (a->dims == b->dims) {
            const int vec = gfh::aligned16(pa) && gfh::aligned16(pb) && gfh::aligned16(pc);
            hipLaunchKernelGGL(binary_same_kernel<OP>, dim3(grid_for(vec ? c->numel / 4 + 1 : c->numel)),
                               dim3(kThreads), 0, nullptr, pa, pb, pc, c->numel, vec);
        } else {
            const std::vector<int64_t> sa = bcast_strides(a->dims, dims), sb = bcast_strides(b->dims, dims);
            // Drop size-1 dims, then merge a dim into the next inner one when
            // both operands are contiguous across the pair.
            Bcast d{};
            d.nd = 0;
            for (size_t i = 0; i < dims.size(); ++i) {
                if (dims[i] == 1) continue;
                if (d.nd > 0) {
                    const int j = d.nd - 1;
                    if (d.sa[j] == sa[i] * (int64_t)dims[i] && d.sb[j] == sb[i] * (int64_t)dims[i]) {
                        d.dim[j] *= (int64_t)dims[i];
                        d.sa[j] = sa[i];
                        d.sb[j] = sb[i];
                        continue;
                    }
                }
                if (d.nd == kMaxDims)
                    return set_error(GFH_COMPUTATION_FAILED, "%s: more than %d broadcast dimensions", name,
                                     kMaxDims);
                d.dim[d.nd] = (int64_t)dims[i];
                d.sa[d.nd] = sa[i];
                d.sb[d.nd] = sb[i];
                ++d.nd;
            }
            if (d.nd == 0) {  // every dim is 1: one element
                d.nd = 1;
                d.dim[0] = 1;
                d.sa[0] = d.sb[0] = 0;
            }
            hipLaunchKernelGGL(binary_bcast_kernel<OP>, dim3(grid_for(c->numel)), dim3(kThreads), 0, nullptr, pa,
                               pb, pc, c->numel, d);
        }
        GFH_TRY(gfh::check_launch(name));
    }
    *out = guard.release();
    return GFH_SUCCESS;
}

int make_filled(const uintptr_t *shape, uintptr_t shape_len, float v, GhostFlowTensor **out) {
    if (!shape || !out) return set_error(GFH_NULL_POINTER, "null shape or out");
    std::vector<size_t> dims(shape, shape + shape_len);
    GhostFlowTensor *t = nullptr;
    GFH_TRY(new_tensor(dims, &t));
    std::unique_ptr<GhostFlowTensor> guard(t);
    if (t->numel > 0) {
        hipLaunchKernelGGL(fill_kernel, dim3(grid_for(t->numel)), dim3(kThreads), 0, nullptr, t->buf->p, t->numel,
                           v);
        GFH_TRY(gfh::check_launch("fill"));
    }
    *out = guard.release();
    return GFH_SUCCESS;
}

template <typename F>
GhostFlowError entry(F &&f) {
    gfh::clear_error();
    try {
        return as_ffi(f());
    } catch (const std::bad_alloc &) {
        return as_ffi(set_error(GFH_ALLOCATION_FAILED, "host allocation failed"));
    } catch (...) {
        return as_ffi(set_error(GFH_UNKNOWN, "unexpected C++ exception"));
    }
}

}  // namespace

extern "C" {

GHOSTFLOW_API GhostFlowError ghostflow_init(void) {
    return entry([] { return gfh::ensure_init(); });
}

GHOSTFLOW_API const char *ghostflow_version(void) {
    const char *v = gfh_version();
    char *s = static_cast<char *>(std::malloc(std::strlen(v) + 1));
    if (s) std::strcpy(s, v);
    return s;
}

GHOSTFLOW_API void ghostflow_free_string(char *s) { std::free(s); }

GHOSTFLOW_API GhostFlowError ghostflow_tensor_create(const float *data, uintptr_t data_len, const uintptr_t *shape,
                                                     uintptr_t shape_len, GhostFlowTensor **out) {
    return entry([&]() -> int {
        if (!data || !shape || !out) return set_error(GFH_NULL_POINTER, "tensor_create: null data, shape or out");
        size_t numel = 0;
        if (!shape_numel(shape, shape_len, &numel) || numel != data_len)
            return set_error(GFH_INVALID_SHAPE, "tensor_create: data length %zu does not match the shape",
                             (size_t)data_len);
        GhostFlowTensor *t = nullptr;
        GFH_TRY(new_tensor(std::vector<size_t>(shape, shape + shape_len), &t));
        std::unique_ptr<GhostFlowTensor> guard(t);
        if (numel > 0) {
            const hipError_t e = hipMemcpy(t->buf->p, data, numel * sizeof(float), hipMemcpyHostToDevice);
            if (e != hipSuccess)
                return set_error(GFH_COMPUTATION_FAILED, "tensor_create: copy to device: %s", hipGetErrorString(e));
        }
        *out = guard.release();
        return GFH_SUCCESS;
    });
}

GHOSTFLOW_API GhostFlowError ghostflow_tensor_zeros(const uintptr_t *shape, uintptr_t shape_len,
                                                    GhostFlowTensor **out) {
    return entry([&] { return make_filled(shape, shape_len, 0.f, out); });
}

GHOSTFLOW_API GhostFlowError ghostflow_tensor_ones(const uintptr_t *shape, uintptr_t shape_len,
                                                   GhostFlowTensor **out) {
    return entry([&] { return make_filled(shape, shape_len, 1.f, out); });
}

GHOSTFLOW_API void ghostflow_tensor_free(GhostFlowTensor *tensor) { delete tensor; }

GHOSTFLOW_API GhostFlowError ghostflow_tensor_shape(const GhostFlowTensor *tensor, uintptr_t *out_shape,
                                                    uintptr_t *out_ndim) {
    return entry([&]() -> int {
        if (!tensor || !out_shape || !out_ndim) return set_error(GFH_NULL_POINTER, "tensor_shape: null argument");
        *out_ndim = tensor->dims.size();
        for (size_t i = 0; i < tensor->dims.size(); ++i) out_shape[i] = tensor->dims[i];
        return GFH_SUCCESS;
    });
}

GHOSTFLOW_API GhostFlowError ghostflow_tensor_data(const GhostFlowTensor *tensor, float *out_data,
                                                   uintptr_t *out_len) {
    return entry([&]() -> int {
        if (!tensor || !out_data || !out_len) return set_error(GFH_NULL_POINTER, "tensor_data: null argument");
        if (tensor->numel > 0) {
            DeviceScope scope(tensor->buf->device);
            if (!scope.ok()) return set_error(GFH_COMPUTATION_FAILED, "tensor_data: cannot select the device");
            const hipError_t e =
                hipMemcpy(out_data, tensor->buf->p, tensor->numel * sizeof(float), hipMemcpyDeviceToHost);
            if (e != hipSuccess)
                return set_error(GFH_COMPUTATION_FAILED, "tensor_data: copy to host: %s", hipGetErrorString(e));
        }
        *out_len = tensor->numel;
        return GFH_SUCCESS;
    });
}

GHOSTFLOW_API GhostFlowError ghostflow_tensor_add(const GhostFlowTensor *a, const GhostFlowTensor *b,
                                                  GhostFlowTensor **out) {
    return entry([&] { return binary<0>(a, b, out, "tensor_add"); });
}

GHOSTFLOW_API GhostFlowError ghostflow_tensor_mul(const GhostFlowTensor *a, const GhostFlowTensor *b,
                                                  GhostFlowTensor **out) {
    return entry([&] { return binary<1>(a, b, out, "tensor_mul"); });
}

GHOSTFLOW_API GhostFlowError ghostflow_tensor_matmul(const GhostFlowTensor *a, const GhostFlowTensor *b,
                                                     GhostFlowTensor **out) {
    return entry([&]() -> int {
        if (!a || !b || !out) return set_error(GFH_NULL_POINTER, "tensor_matmul: null argument");
        // Every failure past the null checks is ComputationFailed, as the
        // reference maps any error of Tensor::matmul (lib.rs:296-301).
        const int rc = [&]() -> int {
            const auto &ad = a->dims, &bd = b->dims;
            if (ad.size() < 2 || bd.size() < 2)
                return set_error(GFH_COMPUTATION_FAILED, "matmul requires at least 2D tensors");
            const size_t m = ad[ad.size() - 2], k = ad.back(), k2 = bd[bd.size() - 2], n = bd.back();
            if (k != k2)
                return set_error(GFH_COMPUTATION_FAILED, "matmul: shape mismatch, expected [%zu, %zu] got [%zu, %zu]",
                                 m, k, k2, n);
            if (a->buf->device != b->buf->device)
                return set_error(GFH_COMPUTATION_FAILED, "matmul: operands on devices %d and %d", a->buf->device,
                                 b->buf->device);
            std::vector<size_t> dims;
            size_t batch = 1, ba = 1, bb = 1;
            if (ad.size() == 2 && bd.size() == 2) {
                dims = {m, n};
            } else {
                const std::vector<size_t> abat(ad.begin(), ad.end() - 2), bbat(bd.begin(), bd.end() - 2);
                if (!broadcast_dims(abat, bbat, &dims))
                    return set_error(GFH_COMPUTATION_FAILED, "matmul: batch dimensions do not broadcast");
                for (size_t d : dims) batch *= d;
                for (size_t d : abat) ba *= d;
                for (size_t d : bbat) bb *= d;
                dims.push_back(m);
                dims.push_back(n);
            }
            DeviceScope scope(a->buf->device);
            if (!scope.ok()) return set_error(GFH_COMPUTATION_FAILED, "matmul: cannot select the device");
            GhostFlowTensor *c = nullptr;
            GFH_TRY(new_tensor(dims, &c));
            std::unique_ptr<GhostFlowTensor> guard(c);
            if (c->numel > 0) {
                const int64_t lda = k > 0 ? (int64_t)k : 1, ldb = (int64_t)n, ldc = (int64_t)n;
                int st;
                if (ad.size() == 2 && bd.size() == 2)
                    st = gfh_sgemm(0, 0, (int64_t)m, (int64_t)n, (int64_t)k, 1.f, a->buf->p, lda, b->buf->p, ldb,
                                   0.f, c->buf->p, ldc, nullptr, nullptr);
                else
                    st = gfh_sgemm_strided_batched(0, 0, (int64_t)m, (int64_t)n, (int64_t)k, 1.f, a->buf->p, lda,
                                                   (int64_t)(m * k), (int64_t)(ba > 0 ? ba : 1), b->buf->p, ldb,
                                                   (int64_t)(k * n), (int64_t)(bb > 0 ? bb : 1), 0.f, c->buf->p,
                                                   ldc, (int64_t)(m * n), (int64_t)batch, nullptr, nullptr);
                if (st != GFH_SUCCESS) return set_error(GFH_COMPUTATION_FAILED, "matmul: %s", gfh::last_error());
            }
            *out = guard.release();
            return GFH_SUCCESS;
        }();
        return rc == GFH_SUCCESS ? rc : GFH_COMPUTATION_FAILED;
    });
}

GHOSTFLOW_API GhostFlowError ghostflow_tensor_reshape(const GhostFlowTensor *tensor, const uintptr_t *new_shape,
                                                      uintptr_t new_shape_len, GhostFlowTensor **out) {
    return entry([&]() -> int {
        if (!tensor || !new_shape || !out) return set_error(GFH_NULL_POINTER, "tensor_reshape: null argument");
        size_t numel = 0;
        if (!shape_numel(new_shape, new_shape_len, &numel) || numel != tensor->numel)
            return set_error(GFH_INVALID_SHAPE, "Cannot reshape tensor of %zu elements to the given shape",
                             tensor->numel);
        std::unique_ptr<GhostFlowTensor> t(new GhostFlowTensor);
        t->dims.assign(new_shape, new_shape + new_shape_len);
        t->numel = numel;
        t->buf = tensor->buf;
        *out = t.release();
        return GFH_SUCCESS;
    });
}

GHOSTFLOW_API const char *ghostflow_get_last_error(void) { return gfh::last_error(); }

}  // extern "C"
