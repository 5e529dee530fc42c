// api.hip -- the extern "C" boundary (include/ghostflow_hip.h).
//
// Every entry point validates its arguments on the host before touching the
// device: sizes and leading dimensions first, then pointers (NULL, and -- with
// pointer checks on -- that each buffer is device memory large enough for
// the access), then lazy device init, then the launch on the caller's
// stream.  No C++ exception crosses the boundary.  Status codes follow
// GhostFlowError (ghostflow-ffi/src/lib.rs:27-35).
#include <algorithm>
#include <climits>
#include <cmath>
#include <initializer_list>
#include <new>

#include "common.hpp"
#include "kernels.hpp"

using namespace gfh;

namespace {

constexpr int64_t kMaxDim = INT32_MAX;

bool mul_ok(int64_t a, int64_t b, int64_t *out) {
    __int128 r = (__int128)a * (__int128)b;
    if (r > (__int128)INT64_MAX / 8) return false;
    *out = (int64_t)r;
    return true;
}

// Whether the product of dims (each >= 0) stays far from int64 / size_t
// overflow, so that byte sizes computed from it are exact.
bool count_ok(std::initializer_list<int64_t> dims) {
    int64_t c = 1;
    for (int64_t d : dims)
        if (!mul_ok(c, d, &c)) return false;
    return true;
}

// Elements spanned by a rows x cols matrix with leading dimension ld.
bool extent2d(int64_t rows, int64_t cols, int64_t ld, int64_t *out) {
    if (rows == 0 || cols == 0) {
        *out = 0;
        return true;
    }
    int64_t t;
    if (!mul_ok(rows - 1, ld, &t)) return false;
    *out = t + cols;
    return true;
}

// Extent of `batch` slices `stride` apart, each `one` elements.
bool extent_batched(int64_t one, int64_t batch, int64_t stride, int64_t *out) {
    if (one == 0 || batch == 0) {
        *out = 0;
        return true;
    }
    int64_t t;
    if (!mul_ok(batch - 1, stride, &t)) return false;
    *out = t + one;
    return true;
}

template <typename F>
int guarded(F &&f) {
    try {
        return f();
    } catch (const std::bad_alloc &) {
        return set_error(GFH_ALLOCATION_FAILED, "host allocation failed");
    } catch (...) {
        return set_error(GFH_UNKNOWN, "unexpected C++ exception");
    }
}

int sgemm_common(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha, const float *a,
                 int64_t lda, int64_t stride_a, int64_t batch_a, const float *b, int64_t ldb, int64_t stride_b,
                 int64_t batch_b, float beta, float *c, int64_t ldc, int64_t stride_c, int64_t batch,
                 const float *bias, gfh_stream_t stream) {
    if (m < 0 || n < 0 || k < 0 || m > kMaxDim || n > kMaxDim || k > kMaxDim)
        return set_error(GFH_INVALID_SHAPE, "sgemm: dims must be in [0, 2^31): m=%lld n=%lld k=%lld", (long long)m,
                         (long long)n, (long long)k);
    if (batch < 0 || batch_a < 1 || batch_b < 1 || batch > 65535)
        return set_error(GFH_INVALID_SHAPE, "sgemm: batch=%lld batch_a=%lld batch_b=%lld out of range",
                         (long long)batch, (long long)batch_a, (long long)batch_b);
    if (stride_a < 0 || stride_b < 0 || stride_c < 0)
        return set_error(GFH_INVALID_SHAPE, "sgemm: negative stride");
    const int64_t a_rows = trans_a ? k : m, a_cols = trans_a ? m : k;
    const int64_t b_rows = trans_b ? n : k, b_cols = trans_b ? k : n;
    if (lda < (a_cols > 0 ? a_cols : 1) || ldb < (b_cols > 0 ? b_cols : 1) || ldc < (n > 0 ? n : 1))
        return set_error(GFH_INVALID_SHAPE, "sgemm: leading dimension too small (lda=%lld ldb=%lld ldc=%lld)",
                         (long long)lda, (long long)ldb, (long long)ldc);
    if (m == 0 || n == 0 || batch == 0) return GFH_SUCCESS;
    int64_t ea, eb, ec, t;
    if (!extent2d(a_rows, a_cols, lda, &t) || !extent_batched(t, batch < batch_a ? batch : batch_a, stride_a, &ea) ||
        !extent2d(b_rows, b_cols, ldb, &t) || !extent_batched(t, batch < batch_b ? batch : batch_b, stride_b, &eb) ||
        !extent2d(m, n, ldc, &t) || !extent_batched(t, batch, stride_c, &ec))
        return set_error(GFH_INVALID_SHAPE, "sgemm: operand extent overflows");
    if (k > 0) {
        GFH_TRY(require_range(a, (size_t)ea * 4, "A"));
        GFH_TRY(require_range(b, (size_t)eb * 4, "B"));
    }
    GFH_TRY(require_range(c, (size_t)ec * 4, "C"));
    GFH_TRY(optional_range(bias, (size_t)n * 4, "bias"));
    GFH_TRY(ensure_init());
    SgemmDesc d;
    d.trans_a = trans_a != 0;
    d.trans_b = trans_b != 0;
    d.m = m;
    d.n = n;
    d.k = k;
    d.alpha = alpha;
    d.beta = beta;
    d.a = a;
    d.lda = lda;
    d.stride_a = stride_a;
    d.batch_a = batch_a;
    d.b = b;
    d.ldb = ldb;
    d.stride_b = stride_b;
    d.batch_b = batch_b;
    d.c = c;
    d.ldc = ldc;
    d.stride_c = stride_c;
    d.batch = batch;
    d.bias = bias;
    return launch_sgemm(d, as_stream(stream));
}

}  // namespace

extern "C" {

GFH_API int gfh_init(void) {
    return guarded([]() -> int { return ensure_init(); });
}

GFH_API int gfh_shutdown(void) {
    return guarded([]() -> int {
        release_stream_state();
        return GFH_SUCCESS;
    });
}

GFH_API const char *gfh_last_error(void) { return last_error(); }

GFH_API const char *gfh_version(void) { return "ghostflow-hip 0.1.0 (gfx950)"; }

GFH_API int gfh_set_pointer_checks(int enabled) { return set_pointer_checks(enabled); }

GFH_API int gfh_sgemm(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha, const float *a,
                      int64_t lda, const float *b, int64_t ldb, float beta, float *c, int64_t ldc,
                      const float *bias, gfh_stream_t stream) {
    return guarded([&]() -> int {
        return sgemm_common(trans_a, trans_b, m, n, k, alpha, a, lda, 0, 1, b, ldb, 0, 1, beta, c, ldc, 0, 1, bias,
                            stream);
    });
}

GFH_API int gfh_sgemm_strided_batched(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha,
                                      const float *a, int64_t lda, int64_t stride_a, int64_t batch_a,
                                      const float *b, int64_t ldb, int64_t stride_b, int64_t batch_b, float beta,
                                      float *c, int64_t ldc, int64_t stride_c, int64_t batch, const float *bias,
                                      gfh_stream_t stream) {
    return guarded([&]() -> int {
        return sgemm_common(trans_a, trans_b, m, n, k, alpha, a, lda, stride_a, batch_a, b, ldb, stride_b, batch_b,
                            beta, c, ldc, stride_c, batch, bias, stream);
    });
}

// grad_a = grad . b^T (NT, K = n) and grad_b = a^T . grad (TN, K = m): the
// two products of matmul_backward (ghostflow-autograd/src/backward.rs:131-160)
// as two validated sgemm launches.
GFH_API int gfh_matmul_backward_f32(const float *grad, const float *a, const float *b, int64_t m, int64_t k,
                                    int64_t n, float *grad_a, float *grad_b, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (m < 0 || k < 0 || n < 0)
            return set_error(GFH_INVALID_SHAPE, "matmul_backward: dims m=%lld k=%lld n=%lld must be >= 0",
                             (long long)m, (long long)k, (long long)n);
        const int64_t ln = std::max<int64_t>(n, 1), lk = std::max<int64_t>(k, 1);
        if (grad_a)
            GFH_TRY(sgemm_common(0, 1, m, k, n, 1.f, grad, ln, 0, 1, b, ln, 0, 1, 0.f, grad_a, lk, 0, 1, nullptr,
                                 stream));
        if (grad_b)
            GFH_TRY(sgemm_common(1, 0, k, n, m, 1.f, a, lk, 0, 1, grad, ln, 0, 1, 0.f, grad_b, ln, 0, 1, nullptr,
                                 stream));
        return GFH_SUCCESS;
    });
}

GFH_API int gfh_quantize_i8_per_channel(const float *x, int64_t rows, int64_t cols, int symmetric, int8_t *q,
                                        float *scales, int8_t *zero_points, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (rows < 0 || cols < 0 || rows > kMaxDim || cols > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "quantize_per_channel: rows=%lld cols=%lld out of range",
                             (long long)rows, (long long)cols);
        if (rows == 0) return GFH_SUCCESS;
        int64_t numel;
        if (!mul_ok(rows, cols, &numel)) return set_error(GFH_INVALID_SHAPE, "quantize_per_channel: overflow");
        GFH_TRY(require_range(x, (size_t)numel * 4, "x"));
        GFH_TRY(require_range(q, (size_t)numel, "q"));
        GFH_TRY(require_range(scales, (size_t)rows * 4, "scales"));
        GFH_TRY(require_range(zero_points, (size_t)rows, "zero_points"));
        GFH_TRY(ensure_init());
        return launch_quantize_per_channel(x, rows, cols, symmetric != 0, q, scales, zero_points,
                                           as_stream(stream));
    });
}

GFH_API size_t gfh_quantize_i8_per_tensor_workspace_size(int64_t n) {
    if (n < 0 || n > ((int64_t)1 << 40)) return 0;
    return quantize_per_tensor_workspace(n);
}

GFH_API int gfh_quantize_i8_per_tensor(const float *x, int64_t n, int symmetric, int8_t *q, float *scale,
                                       int8_t *zero_point, void *workspace, size_t workspace_bytes,
                                       gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (n < 0 || n > ((int64_t)1 << 40))
            return set_error(GFH_INVALID_SHAPE, "quantize_per_tensor: n=%lld out of range", (long long)n);
        GFH_TRY(require_range(x, (size_t)n * 4, "x"));
        GFH_TRY(require_range(q, (size_t)n, "q"));
        GFH_TRY(require_range(scale, 4, "scale"));
        GFH_TRY(require_range(zero_point, 1, "zero_point"));
        GFH_TRY(ensure_init());
        hipStream_t s = as_stream(stream);
        Scratch ws;
        GFH_TRY(ws.acquire(workspace, workspace_bytes, quantize_per_tensor_workspace(n), s));
        return launch_quantize_per_tensor(x, n, symmetric != 0, q, scale, zero_point, ws.ptr(), s);
    });
}

GFH_API int gfh_dequantize_i8(const int8_t *q, int64_t rows, int64_t cols, const float *scales,
                              const int8_t *zero_points, int64_t nscales, float *out, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (rows < 0 || cols < 0 || rows > kMaxDim || cols > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "dequantize: rows=%lld cols=%lld out of range", (long long)rows,
                             (long long)cols);
        if (nscales != 1 && nscales != rows)
            return set_error(GFH_INVALID_SHAPE, "dequantize: nscales=%lld must be 1 or rows=%lld",
                             (long long)nscales, (long long)rows);
        if (rows == 0 || cols == 0) return GFH_SUCCESS;
        int64_t numel;
        if (!mul_ok(rows, cols, &numel)) return set_error(GFH_INVALID_SHAPE, "dequantize: overflow");
        GFH_TRY(require_range(q, (size_t)numel, "q"));
        GFH_TRY(require_range(scales, (size_t)nscales * 4, "scales"));
        GFH_TRY(require_range(zero_points, (size_t)nscales, "zero_points"));
        GFH_TRY(require_range(out, (size_t)numel * 4, "out"));
        GFH_TRY(ensure_init());
        return launch_dequantize(q, rows, cols, scales, zero_points, nscales, out, as_stream(stream));
    });
}

GFH_API int gfh_qweight_rowsum(const int8_t *qw, int64_t n, int64_t k, int32_t *rowsum, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (n < 0 || k < 0 || n > kMaxDim || k > (1 << 24))
            return set_error(GFH_INVALID_SHAPE, "qweight_rowsum: n=%lld k=%lld out of range", (long long)n,
                             (long long)k);
        if (n == 0) return GFH_SUCCESS;
        GFH_TRY(require_range(qw, (size_t)n * (size_t)k, "qw"));
        GFH_TRY(require_range(rowsum, (size_t)n * 4, "rowsum"));
        GFH_TRY(ensure_init());
        return launch_rowsum_i8(qw, n, k, rowsum, as_stream(stream));
    });
}

GFH_API int gfh_qlinear_i8(const int8_t *qx, const float *sx, const int8_t *zx, int x_per_row, const int8_t *qw,
                           const float *sw, const int32_t *w_rowsum, const float *bias, float *y, int32_t *acc_out,
                           int64_t m, int64_t n, int64_t k, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (m < 0 || n < 0 || k < 0 || m > kMaxDim || n > kMaxDim || k > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "qlinear: m=%lld n=%lld k=%lld out of range", (long long)m,
                             (long long)n, (long long)k);
        // |acc| <= 255 * 128 * k must stay below 2^31 for the exact int32 accumulator.
        if (k > 65793)
            return set_error(GFH_INVALID_SHAPE, "qlinear: k=%lld exceeds the exact-int32 bound (65793)",
                             (long long)k);
        if (!y && !acc_out) return set_error(GFH_NULL_POINTER, "qlinear: y and acc_out are both NULL");
        if (zx && !w_rowsum)
            return set_error(GFH_NULL_POINTER, "qlinear: w_rowsum is required when zero points are given");
        if (m == 0 || n == 0) return GFH_SUCCESS;
        int64_t t;
        if (!mul_ok(m, k, &t) || !mul_ok(n, k, &t) || !mul_ok(m, n, &t))
            return set_error(GFH_INVALID_SHAPE, "qlinear: m=%lld n=%lld k=%lld overflow", (long long)m, (long long)n,
                             (long long)k);
        const int64_t nx = x_per_row ? m : 1;
        GFH_TRY(require_range(qx, (size_t)m * (size_t)k, "qx"));
        GFH_TRY(require_range(qw, (size_t)n * (size_t)k, "qw"));
        if (y) {
            GFH_TRY(require_range(sx, (size_t)nx * 4, "sx"));
            GFH_TRY(require_range(sw, (size_t)n * 4, "sw"));
        }
        GFH_TRY(optional_range(zx, (size_t)nx, "zx"));
        GFH_TRY(optional_range(w_rowsum, (size_t)n * 4, "w_rowsum"));
        GFH_TRY(optional_range(bias, (size_t)n * 4, "bias"));
        GFH_TRY(optional_range(y, (size_t)m * (size_t)n * 4, "y"));
        GFH_TRY(optional_range(acc_out, (size_t)m * (size_t)n * 4, "acc_out"));
        GFH_TRY(ensure_init());
        QLinearDesc d;
        d.qx = qx;
        d.sx = sx;
        d.zx = zx;
        d.x_per_row = x_per_row != 0;
        d.qw = qw;
        d.sw = sw;
        d.w_rowsum = w_rowsum;
        d.bias = bias;
        d.y = y;
        d.acc = acc_out;
        d.m = m;
        d.n = n;
        d.k = k;
        return launch_qlinear_i8(d, as_stream(stream));
    });
}

namespace {
// Workspace of gfh_qlinear_dynamic_i8's two-launch form: codes [m*k] | scale,
// zero point | the quantize pass's min/max partials, each 256-byte aligned.
size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }
size_t qdyn_workspace(int64_t m, int64_t k) {
    const size_t mk = (size_t)m * (size_t)k;
    return round256(mk) + 256 + round256(quantize_per_tensor_workspace((int64_t)mk));
}
}  // namespace

GFH_API size_t gfh_qlinear_dynamic_i8_workspace_size(int64_t m, int64_t k) {
    int64_t t;
    if (m <= 0 || k <= 0 || m > kMaxDim || k > kMaxDim || !mul_ok(m, k, &t)) return 0;
    return qdyn_workspace(m, k);
}

GFH_API int gfh_qlinear_dynamic_i8(const float *x, const int8_t *qw, const float *sw, const int32_t *w_rowsum,
                                   const float *bias, float *y, int64_t m, int64_t n, int64_t k, void *workspace,
                                   size_t workspace_bytes, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (m < 0 || n < 0 || k < 0 || m > kMaxDim || n > kMaxDim || k > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "qlinear_dynamic: m=%lld n=%lld k=%lld out of range", (long long)m,
                             (long long)n, (long long)k);
        if (k > 65793)
            return set_error(GFH_INVALID_SHAPE, "qlinear_dynamic: k=%lld exceeds the exact-int32 bound (65793)",
                             (long long)k);
        if (!y || !w_rowsum) return set_error(GFH_NULL_POINTER, "qlinear_dynamic: y and w_rowsum are required");
        if (m == 0 || n == 0) return GFH_SUCCESS;
        int64_t t;
        if (!mul_ok(m, k, &t) || !mul_ok(n, k, &t) || !mul_ok(m, n, &t))
            return set_error(GFH_INVALID_SHAPE, "qlinear_dynamic: m=%lld n=%lld k=%lld overflow", (long long)m,
                             (long long)n, (long long)k);
        GFH_TRY(require_range(x, (size_t)m * (size_t)k * 4, "x"));
        GFH_TRY(require_range(qw, (size_t)n * (size_t)k, "qw"));
        GFH_TRY(require_range(sw, (size_t)n * 4, "sw"));
        GFH_TRY(require_range(w_rowsum, (size_t)n * 4, "w_rowsum"));
        GFH_TRY(optional_range(bias, (size_t)n * 4, "bias"));
        GFH_TRY(require_range(y, (size_t)m * (size_t)n * 4, "y"));
        GFH_TRY(ensure_init());
        hipStream_t s = as_stream(stream);
        QLinearDesc d;
        d.qw = qw;
        d.sw = sw;
        d.w_rowsum = w_rowsum;
        d.bias = bias;
        d.y = y;
        d.m = m;
        d.n = n;
        d.k = k;
        if (qlinear_qx_fits(m, n, k, false) && aligned16(x) && aligned16(qw)) {
            d.xf = x;  // one launch: the INT8 kernel quantizes x itself
            return launch_qlinear_i8(d, s);
        }
        Scratch ws;
        GFH_TRY(ws.acquire(workspace, workspace_bytes, qdyn_workspace(m, k), s));
        char *base = static_cast<char *>(ws.ptr());
        const size_t mk = (size_t)m * (size_t)k;
        int8_t *qx = reinterpret_cast<int8_t *>(base);
        float *sx = reinterpret_cast<float *>(base + round256(mk));
        int8_t *zx = reinterpret_cast<int8_t *>(base + round256(mk) + 4);
        void *part = base + round256(mk) + 256;
        GFH_TRY(launch_quantize_per_tensor(x, (int64_t)mk, false, qx, sx, zx, part, s));
        d.qx = qx;
        d.sx = sx;
        d.zx = zx;
        return launch_qlinear_i8(d, s);
    });
}

GFH_API int gfh_gemv_f32(const float *x, const float *w, float *y, int64_t b, int64_t k, int64_t n,
                         gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (b < 0 || k < 0 || n < 0 || b > 64 || k > kMaxDim || n > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "gemv_f32: b=%lld (<= 64) k=%lld n=%lld out of range",
                             (long long)b, (long long)k, (long long)n);
        if (b == 0 || n == 0) return GFH_SUCCESS;
        if (!count_ok({k, n}))
            return set_error(GFH_INVALID_SHAPE, "gemv: k=%lld n=%lld overflow", (long long)k, (long long)n);
        GFH_TRY(require_range(x, (size_t)b * (size_t)k * 4, "x"));
        GFH_TRY(require_range(w, (size_t)k * (size_t)n * 4, "w"));
        GFH_TRY(require_range(y, (size_t)b * (size_t)n * 4, "y"));
        GFH_TRY(ensure_init());
        return launch_gemv_f32(x, w, y, b, k, n, as_stream(stream));
    });
}

GFH_API int gfh_gemv_w8(const float *x, const int8_t *qw, const float *scales, const int8_t *zero_points, float *y,
                        int64_t b, int64_t k, int64_t n, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (b < 0 || k < 0 || n < 0 || b > 64 || k > kMaxDim || n > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "gemv_w8: b=%lld (<= 64) k=%lld n=%lld out of range",
                             (long long)b, (long long)k, (long long)n);
        if (b == 0 || n == 0) return GFH_SUCCESS;
        if (!count_ok({k, n}))
            return set_error(GFH_INVALID_SHAPE, "gemv: k=%lld n=%lld overflow", (long long)k, (long long)n);
        GFH_TRY(require_range(x, (size_t)b * (size_t)k * 4, "x"));
        GFH_TRY(require_range(qw, (size_t)k * (size_t)n, "qw"));
        GFH_TRY(require_range(scales, (size_t)k * 4, "scales"));
        GFH_TRY(optional_range(zero_points, (size_t)k, "zero_points"));
        GFH_TRY(require_range(y, (size_t)b * (size_t)n * 4, "y"));
        GFH_TRY(ensure_init());
        return launch_gemv_w8(x, qw, scales, zero_points, y, b, k, n, as_stream(stream));
    });
}

GFH_API int gfh_gemv_w8_noalloc(const float *x, const int8_t *qw, const float *scales, const int8_t *zero_points,
                                float *y, int64_t b, int64_t k, int64_t n, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (b < 0 || k < 0 || n < 0 || b > 64 || k > kMaxDim || n > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "gemv_w8_noalloc: b=%lld (<= 64) k=%lld n=%lld out of range",
                             (long long)b, (long long)k, (long long)n);
        if (b == 0 || n == 0) return GFH_SUCCESS;
        if (!count_ok({k, n}))
            return set_error(GFH_INVALID_SHAPE, "gemv: k=%lld n=%lld overflow", (long long)k, (long long)n);
        GFH_TRY(require_range(x, (size_t)b * (size_t)k * 4, "x"));
        GFH_TRY(require_range(qw, (size_t)k * (size_t)n, "qw"));
        GFH_TRY(require_range(scales, (size_t)k * 4, "scales"));
        GFH_TRY(optional_range(zero_points, (size_t)k, "zero_points"));
        GFH_TRY(require_range(y, (size_t)b * (size_t)n * 4, "y"));
        GFH_TRY(ensure_init());
        return launch_gemv_w8_noalloc(x, qw, scales, zero_points, y, b, k, n, as_stream(stream));
    });
}

GFH_API int gfh_softmax_lastdim_f32(const float *x, float *y, int64_t rows, int64_t cols, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (rows < 0 || cols < 0 || rows > kMaxDim || cols > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "softmax: rows=%lld cols=%lld out of range", (long long)rows,
                             (long long)cols);
        if (rows == 0 || cols == 0) return GFH_SUCCESS;
        int64_t numel;
        if (!mul_ok(rows, cols, &numel)) return set_error(GFH_INVALID_SHAPE, "softmax: overflow");
        GFH_TRY(require_range(x, (size_t)numel * 4, "x"));
        GFH_TRY(require_range(y, (size_t)numel * 4, "y"));
        GFH_TRY(ensure_init());
        return launch_softmax_lastdim(x, y, rows, cols, as_stream(stream));
    });
}

GFH_API size_t gfh_flash_attention_workspace_size(int64_t batch, int64_t seq_len_q, int64_t seq_len_k) {
    if (batch <= 0 || seq_len_q <= 0 || seq_len_k <= 0 || batch > kMaxDim || seq_len_q > kMaxDim ||
        seq_len_k > kMaxDim)
        return 0;
    int64_t t, u;
    if (!mul_ok(batch, seq_len_q, &t) || !mul_ok(t, seq_len_k, &u)) return 0;
    return (size_t)u * sizeof(float);
}

GFH_API int gfh_flash_attention_f32(const float *q, const float *k, const float *v, float *out, int64_t batch,
                                    int64_t seq_len_q, int64_t seq_len_k, int64_t d_model, int64_t block_size_m,
                                    int64_t block_size_n, int causal, float scale, void *workspace,
                                    size_t workspace_bytes, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (batch < 0 || seq_len_q < 0 || seq_len_k < 0 || d_model < 0 || batch > kMaxDim ||
            seq_len_q > kMaxDim || seq_len_k > kMaxDim || d_model > kMaxDim)
            return set_error(GFH_INVALID_SHAPE,
                             "flash_attention: batch=%lld seq_len_q=%lld seq_len_k=%lld d_model=%lld out of range",
                             (long long)batch, (long long)seq_len_q, (long long)seq_len_k, (long long)d_model);
        if (block_size_m <= 0 || block_size_n <= 0)
            return set_error(GFH_INVALID_SHAPE, "flash_attention: block sizes must be positive (m=%lld n=%lld)",
                             (long long)block_size_m, (long long)block_size_n);
        const int64_t nb = seq_len_k > 0 ? (seq_len_k + block_size_n - 1) / block_size_n : 0;
        if (nb > flash_attention_max_blocks())
            return set_error(GFH_INVALID_SHAPE,
                             "flash_attention: seq_len_k / block_size_n = %lld key blocks; at most %lld are served",
                             (long long)nb, (long long)flash_attention_max_blocks());
        int64_t rows, qn, kn, sn;
        if (!mul_ok(batch, seq_len_q, &rows) || rows > (int64_t)INT32_MAX || !mul_ok(rows, d_model, &qn) ||
            !mul_ok(batch, seq_len_k, &kn) || !mul_ok(kn, d_model, &kn) || !mul_ok(rows, seq_len_k, &sn))
            return set_error(GFH_INVALID_SHAPE, "flash_attention: size overflow");
        if (qn == 0) return GFH_SUCCESS;
        GFH_TRY(require_range(q, (size_t)qn * 4, "q"));
        GFH_TRY(require_range(k, (size_t)kn * 4, "k"));
        GFH_TRY(require_range(v, (size_t)kn * 4, "v"));
        GFH_TRY(require_range(out, (size_t)qn * 4, "out"));
        GFH_TRY(ensure_init());
        hipStream_t s = as_stream(stream);
        FlashAttnDesc d;
        d.q = q;
        d.k = k;
        d.v = v;
        d.out = out;
        d.batch = batch;
        d.sq = seq_len_q;
        d.sk = seq_len_k;
        d.d = d_model;
        d.block_m = block_size_m;
        d.block_n = block_size_n;
        d.causal = causal != 0;
        d.scale = scale;
        if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 7) != 0)
            return set_error(GFH_INVALID_DATA, "flash_attention: workspace must be 8-byte aligned");
        Scratch ws;
        GFH_TRY(ws.acquire(workspace, workspace_bytes, flash_attention_workspace_bytes(d), s));
        d.ws = static_cast<float *>(ws.ptr());
        return launch_flash_attention_blockwise(d, s);
    });
}

GFH_API int gfh_sdpa_f32(const float *q, const float *k, const float *v, float *out, float *weights, int64_t b,
                         int64_t h, int64_t sq, int64_t skv, int64_t d, float scale, int causal, const float *mask,
                         int64_t mask_numel, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (b < 0 || h < 0 || sq < 0 || skv < 0 || d < 0 || b > 65535 || h > 65535 || sq > 65535 * 128 ||
            skv > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "sdpa: b=%lld h=%lld sq=%lld skv=%lld out of range", (long long)b,
                             (long long)h, (long long)sq, (long long)skv);
        if (d == 0 || d > 128 || d % 4 != 0)
            return set_error(GFH_INVALID_SHAPE, "sdpa: head_dim %lld must be a multiple of 4 in [4, 128]",
                             (long long)d);
        if (causal && sq != skv)
            return set_error(GFH_INVALID_SHAPE,
                             "sdpa: causal attention needs sq == skv (got %lld, %lld); the top-left causal rule of "
                             "FlashAttention::forward for sq != skv is gfh_flash_attention_f32",
                             (long long)sq, (long long)skv);
        if (mask && (mask_numel <= 0 || !count_ok({mask_numel})))
            return set_error(GFH_INVALID_SHAPE, "sdpa: mask_numel=%lld out of range", (long long)mask_numel);
        if (b == 0 || h == 0 || sq == 0) return GFH_SUCCESS;
        if (skv == 0) return set_error(GFH_INVALID_SHAPE, "sdpa: empty key sequence");
        if (!count_ok({b, h, sq, skv}) || !count_ok({b, h, skv, d}))
            return set_error(GFH_INVALID_SHAPE, "sdpa: b=%lld h=%lld sq=%lld skv=%lld overflow", (long long)b,
                             (long long)h, (long long)sq, (long long)skv);
        const size_t bh = (size_t)b * (size_t)h;
        GFH_TRY(require_range(q, bh * (size_t)sq * (size_t)d * 4, "q"));
        GFH_TRY(require_range(k, bh * (size_t)skv * (size_t)d * 4, "k"));
        GFH_TRY(require_range(v, bh * (size_t)skv * (size_t)d * 4, "v"));
        GFH_TRY(require_range(out, bh * (size_t)sq * (size_t)d * 4, "out"));
        GFH_TRY(optional_range(weights, bh * (size_t)sq * (size_t)skv * 4, "weights"));
        GFH_TRY(optional_range(mask, (size_t)mask_numel * 4, "mask"));
        GFH_TRY(ensure_init());
        SdpaDesc sd;
        sd.q = q;
        sd.k = k;
        sd.v = v;
        sd.out = out;
        sd.weights = weights;
        sd.b = b;
        sd.h = h;
        sd.sq = sq;
        sd.skv = skv;
        sd.d = d;
        sd.scale = scale;
        sd.causal = causal != 0;
        sd.mask = mask;
        sd.mask_numel = mask ? mask_numel : 0;
        return launch_sdpa(sd, as_stream(stream));
    });
}

GFH_API int gfh_kv_attention_f32(const float *q, int64_t ldq, const float *k, const float *v, int64_t capacity,
                                 int64_t ldkv, float *out, int64_t ldo, float *weights, int64_t b, int64_t h,
                                 int64_t sq, int64_t kv_len, int64_t d, float scale, int causal, const float *mask,
                                 int64_t mask_numel, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (b < 0 || h < 0 || sq < 0 || kv_len < 0 || capacity < 0 || b > 65535 || h > 65535 || sq > kMaxDim ||
            kv_len > kMaxDim || capacity > kMaxDim)
            return set_error(GFH_INVALID_SHAPE, "kv_attention: b=%lld h=%lld sq=%lld kv_len=%lld out of range",
                             (long long)b, (long long)h, (long long)sq, (long long)kv_len);
        if (d <= 0 || d > 128 || d % 4 != 0)
            return set_error(GFH_INVALID_SHAPE, "kv_attention: head_dim %lld must be a multiple of 4 in [4, 128]",
                             (long long)d);
        if (kv_len > capacity)
            return set_error(GFH_INVALID_SHAPE, "kv_attention: kv_len %lld exceeds the cache capacity %lld",
                             (long long)kv_len, (long long)capacity);
        const int64_t hd = h * d;
        if (ldq < hd || ldkv < hd || ldo < hd || ldq % 4 || ldkv % 4 || ldo % 4)
            return set_error(GFH_INVALID_SHAPE,
                             "kv_attention: ldq=%lld ldkv=%lld ldo=%lld must be multiples of 4 and >= h*d=%lld",
                             (long long)ldq, (long long)ldkv, (long long)ldo, (long long)hd);
        if (causal && kv_len < sq)
            return set_error(GFH_INVALID_SHAPE, "kv_attention: causal needs kv_len >= sq (got %lld < %lld)",
                             (long long)kv_len, (long long)sq);
        if (mask && (mask_numel <= 0 || !count_ok({mask_numel})))
            return set_error(GFH_INVALID_SHAPE, "kv_attention: mask_numel=%lld out of range", (long long)mask_numel);
        if (b == 0 || h == 0 || sq == 0) return GFH_SUCCESS;
        if (kv_len == 0) return set_error(GFH_INVALID_SHAPE, "kv_attention: empty key sequence");
        int64_t bs, bhs, eq, ekv, eo, ew, t, one;
        if (!mul_ok(b, sq, &bs) || !mul_ok(bs, h, &bhs) || !extent2d(bs, hd, ldq, &eq) ||
            !extent2d(bs, hd, ldo, &eo) || !mul_ok(capacity, ldkv, &t) || !extent2d(kv_len, hd, ldkv, &one) ||
            !extent_batched(one, b, t, &ekv) || !mul_ok(bhs, kv_len, &ew) || !count_ok({sq, ldq}) ||
            !count_ok({sq, ldo}))
            return set_error(GFH_INVALID_SHAPE, "kv_attention: operand extent overflows");
        GFH_TRY(require_range(q, (size_t)eq * 4, "q"));
        GFH_TRY(require_range(k, (size_t)ekv * 4, "k"));
        GFH_TRY(require_range(v, (size_t)ekv * 4, "v"));
        GFH_TRY(require_range(out, (size_t)eo * 4, "out"));
        GFH_TRY(optional_range(weights, (size_t)ew * 4, "weights"));
        GFH_TRY(optional_range(mask, (size_t)mask_numel * 4, "mask"));
        if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
            return set_error(GFH_INVALID_DATA, "kv_attention: q, k, v and out must be 16-byte aligned");
        GFH_TRY(ensure_init());
        KvAttnDesc kd;
        kd.q = q;
        kd.k = k;
        kd.v = v;
        kd.out = out;
        kd.weights = weights;
        kd.mask = mask;
        kd.mask_numel = mask ? mask_numel : 0;
        kd.q_bs = sq * ldq;
        kd.q_rs = ldq;
        kd.kv_bs = t;
        kd.kv_rs = ldkv;
        kd.o_bs = sq * ldo;
        kd.o_rs = ldo;
        kd.b = b;
        kd.h = h;
        kd.sq = sq;
        kd.kv_len = kv_len;
        kd.d = d;
        kd.scale = scale;
        kd.causal = causal != 0;
        return launch_kv_attention(kd, as_stream(stream));
    });
}

GFH_API size_t gfh_mha_workspace_size(int64_t b, int64_t sq, int64_t e) {
    if (b <= 0 || sq <= 0 || e <= 0 || b > 65535 || sq > kMaxDim || e > kMaxDim) return 0;
    return mha_workspace_bytes(b, sq, e);
}

GFH_API int gfh_mha_forward_with_cache_f32(const float *query, const float *key, const float *value, const float *wq,
                                           const float *bq, const float *wk, const float *bk, const float *wv,
                                           const float *bv, const float *wo, const float *bo, float *k_cache,
                                           float *v_cache, int64_t capacity, int64_t past_len, const float *mask,
                                           int64_t mask_numel, int causal, float *out, float *weights, int64_t b,
                                           int64_t sq, int64_t sk, int64_t e, int64_t h, void *workspace,
                                           size_t workspace_bytes, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (b < 0 || sq < 0 || sk < 0 || e < 0 || h <= 0 || past_len < 0 || capacity < 0 || b > 65535 ||
            h > 65535 || sq > kMaxDim || sk > kMaxDim || e > kMaxDim || past_len > kMaxDim || capacity > kMaxDim)
            return set_error(GFH_INVALID_SHAPE,
                             "mha: b=%lld sq=%lld sk=%lld e=%lld h=%lld past_len=%lld capacity=%lld out of range",
                             (long long)b, (long long)sq, (long long)sk, (long long)e, (long long)h,
                             (long long)past_len, (long long)capacity);
        if (e % h != 0)
            return set_error(GFH_INVALID_SHAPE, "mha: embed_dim %lld must be divisible by num_heads %lld",
                             (long long)e, (long long)h);
        const int64_t hd = e / h;
        if (hd < 4 || hd > 128 || hd % 4 != 0)
            return set_error(GFH_INVALID_SHAPE, "mha: head_dim %lld must be a multiple of 4 in [4, 128]",
                             (long long)hd);
        if (past_len + sk > capacity)
            return set_error(GFH_INVALID_SHAPE, "mha: past_len %lld + %lld new keys exceed the cache capacity %lld",
                             (long long)past_len, (long long)sk, (long long)capacity);
        const int64_t kv_len = past_len + sk;
        if (causal && kv_len < sq)
            return set_error(GFH_INVALID_SHAPE, "mha: causal needs past_len + sk >= sq");
        if (mask && (mask_numel <= 0 || !count_ok({mask_numel})))
            return set_error(GFH_INVALID_SHAPE, "mha: mask_numel=%lld out of range", (long long)mask_numel);
        if (b == 0 || sq == 0) return GFH_SUCCESS;
        if (kv_len == 0) return set_error(GFH_INVALID_SHAPE, "mha: empty key sequence");
        int64_t bsq, bsk, ww, cache, bh, bhs, wts;
        if (!mul_ok(b * sq, e, &bsq) || !mul_ok(b * sk, e, &bsk) || !mul_ok(e, e, &ww) ||
            !mul_ok(b * capacity, e, &cache) || !mul_ok(b, h, &bh) || !mul_ok(bh, sq, &bhs) ||
            !mul_ok(bhs, kv_len, &wts))
            return set_error(GFH_INVALID_SHAPE, "mha: operand extent overflows");
        GFH_TRY(require_range(query, (size_t)bsq * 4, "query"));
        GFH_TRY(require_range(key, (size_t)bsk * 4, "key"));
        GFH_TRY(require_range(value, (size_t)bsk * 4, "value"));
        GFH_TRY(require_range(wq, (size_t)ww * 4, "wq"));
        GFH_TRY(require_range(wk, (size_t)ww * 4, "wk"));
        GFH_TRY(require_range(wv, (size_t)ww * 4, "wv"));
        GFH_TRY(require_range(wo, (size_t)ww * 4, "wo"));
        GFH_TRY(optional_range(bq, (size_t)e * 4, "bq"));
        GFH_TRY(optional_range(bk, (size_t)e * 4, "bk"));
        GFH_TRY(optional_range(bv, (size_t)e * 4, "bv"));
        GFH_TRY(optional_range(bo, (size_t)e * 4, "bo"));
        GFH_TRY(require_range(k_cache, (size_t)cache * 4, "k_cache"));
        GFH_TRY(require_range(v_cache, (size_t)cache * 4, "v_cache"));
        GFH_TRY(require_range(out, (size_t)bsq * 4, "out"));
        GFH_TRY(optional_range(weights, (size_t)wts * 4, "weights"));
        GFH_TRY(optional_range(mask, (size_t)mask_numel * 4, "mask"));
        if (!aligned16(k_cache) || !aligned16(v_cache) || (workspace && !aligned16(workspace)))
            return set_error(GFH_INVALID_DATA, "mha: k_cache, v_cache and the workspace must be 16-byte aligned");
        GFH_TRY(ensure_init());
        hipStream_t s = as_stream(stream);
        Scratch ws;
        GFH_TRY(ws.acquire(workspace, workspace_bytes, mha_workspace_bytes(b, sq, e), s));
        MhaDesc d;
        d.query = query;
        d.key = key;
        d.value = value;
        d.wq = wq;
        d.bq = bq;
        d.wk = wk;
        d.bk = bk;
        d.wv = wv;
        d.bv = bv;
        d.wo = wo;
        d.bo = bo;
        d.k_cache = k_cache;
        d.v_cache = v_cache;
        d.capacity = capacity;
        d.past_len = past_len;
        d.mask = mask;
        d.mask_numel = mask ? mask_numel : 0;
        d.causal = causal != 0;
        d.out = out;
        d.weights = weights;
        d.b = b;
        d.sq = sq;
        d.sk = sk;
        d.e = e;
        d.h = h;
        d.scale = 1.0f / sqrtf((float)hd);
        return launch_mha_forward(d, ws.ptr(), s);
    });
}

GFH_API int gfh_silu_mul_f32(const float *gate, const float *up, float *out, int64_t n, gfh_stream_t stream) {
    return guarded([&]() -> int {
        if (n < 0 || n > ((int64_t)1 << 40))
            return set_error(GFH_INVALID_SHAPE, "silu_mul: n=%lld out of range", (long long)n);
        if (n == 0) return GFH_SUCCESS;
        GFH_TRY(require_range(gate, (size_t)n * 4, "gate"));
        GFH_TRY(require_range(up, (size_t)n * 4, "up"));
        GFH_TRY(require_range(out, (size_t)n * 4, "out"));
        GFH_TRY(ensure_init());
        return launch_silu_mul(gate, up, out, n, as_stream(stream));
    });
}

namespace {
// SwiGLU dims in [0, INT32_MAX] whose operand element counts (m x hidden,
// m x inter, hidden x inter) stay far from overflow.
bool swiglu_dims_ok(int64_t m, int64_t hidden, int64_t inter, int64_t *mh, int64_t *mi, int64_t *wi) {
    return m >= 0 && hidden >= 0 && inter >= 0 && m <= kMaxDim && hidden <= kMaxDim && inter <= kMaxDim &&
           mul_ok(m, hidden, mh) && mul_ok(m, inter, mi) && mul_ok(hidden, inter, wi);
}

// Shape checks shared by both SwiGLU entry points.
int swiglu_shapes(const char *what, int64_t m, int64_t hidden, int64_t inter, int64_t *mh, int64_t *mi,
                  int64_t *wi) {
    if (!swiglu_dims_ok(m, hidden, inter, mh, mi, wi))
        return set_error(GFH_INVALID_SHAPE, "%s: m=%lld hidden=%lld inter=%lld out of range", what, (long long)m,
                         (long long)hidden, (long long)inter);
    return GFH_SUCCESS;
}
}  // namespace

GFH_API size_t gfh_swiglu_f32_workspace_size(int64_t m, int64_t inter) {
    int64_t a, b, c;
    if (!swiglu_dims_ok(m, 0, inter, &a, &b, &c)) return 0;
    return swiglu_f32_workspace_bytes(m, inter);
}

GFH_API int gfh_swiglu_f32(const float *x, int64_t m, int64_t hidden, int64_t inter, const float *wg,
                           const float *bg, const float *wu, const float *bu, const float *wd, const float *bd,
                           float *y, float *h, void *workspace, size_t workspace_bytes, gfh_stream_t stream) {
    return guarded([&]() -> int {
        int64_t mh, mi, wi;
        GFH_TRY(swiglu_shapes("swiglu", m, hidden, inter, &mh, &mi, &wi));
        if (m == 0 || hidden == 0) return GFH_SUCCESS;
        GFH_TRY(require_range(x, (size_t)mh * 4, "x"));
        GFH_TRY(require_range(wg, (size_t)wi * 4, "wg"));
        GFH_TRY(require_range(wu, (size_t)wi * 4, "wu"));
        GFH_TRY(require_range(wd, (size_t)wi * 4, "wd"));
        GFH_TRY(optional_range(bg, (size_t)inter * 4, "bg"));
        GFH_TRY(optional_range(bu, (size_t)inter * 4, "bu"));
        GFH_TRY(optional_range(bd, (size_t)hidden * 4, "bd"));
        GFH_TRY(require_range(y, (size_t)mh * 4, "y"));
        GFH_TRY(optional_range(h, (size_t)mi * 4, "h"));
        if (workspace && !aligned16(workspace))
            return set_error(GFH_INVALID_DATA, "swiglu: the workspace must be 16-byte aligned");
        GFH_TRY(ensure_init());
        hipStream_t s = as_stream(stream);
        Scratch ws;
        GFH_TRY(ws.acquire(workspace, workspace_bytes, swiglu_f32_workspace_bytes(m, inter), s));
        SwigluDesc d;
        d.x = x;
        d.m = m;
        d.hidden = hidden;
        d.inter = inter;
        d.wg = wg;
        d.bg = bg;
        d.wu = wu;
        d.bu = bu;
        d.wd = wd;
        d.bd = bd;
        d.y = y;
        d.h = h;
        return launch_swiglu_f32(d, ws.ptr(), s);
    });
}

GFH_API size_t gfh_swiglu_i8_workspace_size(int64_t m, int64_t hidden, int64_t inter) {
    int64_t a, b, c;
    if (!swiglu_dims_ok(m, hidden, inter, &a, &b, &c)) return 0;
    return swiglu_i8_workspace_bytes(m, hidden, inter);
}

GFH_API int gfh_swiglu_i8(const float *x, int64_t m, int64_t hidden, int64_t inter, const int8_t *qwg,
                          const float *swg, const int32_t *rsg, const float *bg, const int8_t *qwu, const float *swu,
                          const int32_t *rsu, const float *bu, const int8_t *qwd, const float *swd,
                          const int32_t *rsd, const float *bd, float *y, float *h, void *workspace,
                          size_t workspace_bytes, gfh_stream_t stream) {
    return guarded([&]() -> int {
        int64_t mh, mi, wi;
        GFH_TRY(swiglu_shapes("swiglu_i8", m, hidden, inter, &mh, &mi, &wi));
        if (hidden % 16 != 0 || inter % 16 != 0)
            return set_error(GFH_INVALID_SHAPE, "swiglu_i8: hidden=%lld and inter=%lld must be multiples of 16",
                             (long long)hidden, (long long)inter);
        if (hidden > 65793 || inter > 65793)
            return set_error(GFH_INVALID_SHAPE, "swiglu_i8: hidden / inter exceed the exact-int32 bound (65793)");
        if (m == 0 || hidden == 0) return GFH_SUCCESS;
        if (inter == 0) return set_error(GFH_INVALID_SHAPE, "swiglu_i8: inter must be > 0");
        GFH_TRY(require_range(x, (size_t)mh * 4, "x"));
        GFH_TRY(require_range(qwg, (size_t)wi, "qwg"));
        GFH_TRY(require_range(qwu, (size_t)wi, "qwu"));
        GFH_TRY(require_range(qwd, (size_t)wi, "qwd"));
        GFH_TRY(require_range(swg, (size_t)inter * 4, "swg"));
        GFH_TRY(require_range(swu, (size_t)inter * 4, "swu"));
        GFH_TRY(require_range(swd, (size_t)hidden * 4, "swd"));
        GFH_TRY(require_range(rsg, (size_t)inter * 4, "rsg"));
        GFH_TRY(require_range(rsu, (size_t)inter * 4, "rsu"));
        GFH_TRY(require_range(rsd, (size_t)hidden * 4, "rsd"));
        GFH_TRY(optional_range(bg, (size_t)inter * 4, "bg"));
        GFH_TRY(optional_range(bu, (size_t)inter * 4, "bu"));
        GFH_TRY(optional_range(bd, (size_t)hidden * 4, "bd"));
        GFH_TRY(require_range(y, (size_t)mh * 4, "y"));
        GFH_TRY(optional_range(h, (size_t)mi * 4, "h"));
        if (!aligned16(qwg) || !aligned16(qwu) || !aligned16(qwd) || (workspace && !aligned16(workspace)))
            return set_error(GFH_INVALID_DATA, "swiglu_i8: weight codes and the workspace must be 16-byte aligned");
        GFH_TRY(ensure_init());
        hipStream_t s = as_stream(stream);
        Scratch ws;
        GFH_TRY(ws.acquire(workspace, workspace_bytes, swiglu_i8_workspace_bytes(m, hidden, inter), s));
        SwigluDesc d;
        d.x = x;
        d.m = m;
        d.hidden = hidden;
        d.inter = inter;
        d.qwg = qwg;
        d.swg = swg;
        d.rsg = rsg;
        d.bg = bg;
        d.qwu = qwu;
        d.swu = swu;
        d.rsu = rsu;
        d.bu = bu;
        d.qwd = qwd;
        d.swd = swd;
        d.rsd = rsd;
        d.bd = bd;
        d.y = y;
        d.h = h;
        return launch_swiglu_i8(d, ws.ptr(), s);
    });
}

}  // extern "C"
