// swiglu.hip -- the LLaMA / Mistral feed-forward block, SwiGLU::forward
// (ghostflow-nn/src/llama.rs:259-287), on one stream:
//
//   gate = x . Wg^T + bg          up = x . Wu^T + bu        [m, inter]
//   h    = silu(gate) * up        silu(v) = v / (1 + exp(-v))
//                                 (activation.rs:117-122; mul, arithmetic.rs:39-45)
//   y    = h . Wd^T + bd                                     [m, hidden]
//
// in fp32 (the reference's own layer: three launch_sgemm NT calls around the
// silu * up kernel) and in int8 (every Linear as the INT8 linear on
// DynamicQuantization's scheme, quantization.rs:251-288: per-channel
// symmetric weight codes, activations x and h quantized per tensor,
// asymmetric, on the device; at m <= 4 inside the two INT8 launches).
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

// silu and the product are separate f32 roundings, as the reference
// computes them (rustc never contracts to FMA).
#pragma clang fp contract(off)

namespace gfh {
namespace {

// out[i] = silu(gate[i]) * up[i]; 16-byte vectors when every pointer allows.
template <bool VEC>
__global__ __launch_bounds__(256) void silu_mul_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                       float *__restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        const int64_t n4 = n / 4;
        for (; i < n4; i += stride) {
            const f32x4 gv = reinterpret_cast<const f32x4 *>(g)[i];
            const f32x4 uv = reinterpret_cast<const f32x4 *>(u)[i];
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = silu_mul1(gv[e], uv[e]);
            reinterpret_cast<f32x4 *>(out)[i] = o;
        }
        i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    }
    for (; i < n; i += stride) out[i] = silu_mul1(g[i], u[i]);
}

constexpr size_t kAlign = 256;
size_t round_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

}  // namespace

int launch_silu_mul(const float *g, const float *u, float *out, int64_t n, hipStream_t s) {
    if (n <= 0) return GFH_SUCCESS;
    const bool vec = aligned16(g) && aligned16(u) && aligned16(out);
    const int64_t work = vec ? (n + 3) / 4 : n;
    const unsigned blocks = (unsigned)std::min<int64_t>((work + 255) / 256, 4096);
    if (vec)
        hipLaunchKernelGGL(silu_mul_kernel<true>, dim3(blocks), dim3(256), 0, s, g, u, out, n);
    else
        hipLaunchKernelGGL(silu_mul_kernel<false>, dim3(blocks), dim3(256), 0, s, g, u, out, n);
    return check_launch("silu_mul");
}

size_t swiglu_f32_workspace_bytes(int64_t m, int64_t inter) {
    return 2 * round_up((size_t)m * (size_t)inter * 4);
}

// fp32: gate and up into the workspace, h over gate (or into d.h), then down.
// Each product is a launch_sgemm NT call (gate and up as one grouped launch
// when m <= 64).
int launch_swiglu_f32(const SwigluDesc &d, void *workspace, hipStream_t s) {
    const size_t one = round_up((size_t)d.m * (size_t)d.inter * 4);
    float *gate = static_cast<float *>(workspace);
    float *up = reinterpret_cast<float *>(static_cast<char *>(workspace) + one);
    float *h = d.h ? d.h : gate;
    auto linear = [&](const float *x, const float *w, const float *bias, float *y, int64_t n, int64_t k) {
        SgemmDesc g;
        g.trans_b = true;
        g.m = d.m;
        g.n = n;
        g.k = k;
        g.a = x;
        g.lda = k;
        g.b = w;
        g.ldb = k;
        g.c = y;
        g.ldc = n;
        g.bias = bias;
        return g;
    };
    // Gate and up read the same x: up to 64 rows they share one grouped
    // launch, otherwise one launch each.
    const SgemmDesc gu[2] = {linear(d.x, d.wg, d.bg, gate, d.inter, d.hidden),
                             linear(d.x, d.wu, d.bu, up, d.inter, d.hidden)};
    if (sgemm_nt_group_fits(gu, 2)) {
        GFH_TRY(launch_sgemm_nt_group(gu, 2, s));
    } else {
        GFH_TRY(launch_sgemm(gu[0], s));
        GFH_TRY(launch_sgemm(gu[1], s));
    }
    GFH_TRY(launch_silu_mul(gate, up, h, d.m * d.inter, s));
    return launch_sgemm(linear(h, d.wd, d.bd, d.y, d.hidden, d.inter), s);
}

// Workspace of the int8 block, each region 256-byte aligned:
//   qx [m*hidden] i8 | sx, zx | x min/max partials |
//   gate (= h) [m*inter] f32 | up [m*inter] f32, unfused path only |
//   qh [m*inter] i8 | sh, zh | h min/max partials
namespace {
// (min, max) partials of h: the fused launch's or the full quantize pass's.
size_t h_partials_bytes(int64_t m, int64_t inter) {
    return std::max(sizeof(float2) * (size_t)qlinear_swiglu_partials(m, inter),
                    quantize_per_tensor_workspace(m * inter));
}
}  // namespace

size_t swiglu_i8_workspace_bytes(int64_t m, int64_t hidden, int64_t inter) {
    const size_t mh = (size_t)m * (size_t)hidden, mi = (size_t)m * (size_t)inter;
    const bool fused = qlinear_swiglu_fits(m, inter, hidden);
    return round_up(mh) + kAlign + round_up(quantize_per_tensor_workspace((int64_t)mh)) +
           (fused ? 1 : 2) * round_up(mi * 4) + round_up(mi) + kAlign + round_up(h_partials_bytes(m, inter));
}

// x -> quantize (per tensor, asymmetric: quantize_activation,
// quantization.rs:280-287) -> gate/up with silu * up in one launch, its
// (min, max) partials feeding the quantize pass of h directly -> down.
// Shapes the fused launch does not serve run gate and up as two INT8
// linears, the silu * up kernel and the full per-tensor quantize of h.
int launch_swiglu_i8(const SwigluDesc &d, void *workspace, hipStream_t s) {
    const size_t mh = (size_t)d.m * (size_t)d.hidden, mi = (size_t)d.m * (size_t)d.inter;
    const bool fused = qlinear_swiglu_fits(d.m, d.inter, d.hidden);
    char *p = static_cast<char *>(workspace);
    auto take = [&](size_t bytes) {
        char *r = p;
        p += round_up(bytes);
        return r;
    };
    int8_t *qx = reinterpret_cast<int8_t *>(take(mh));
    char *xs = take(kAlign);
    float *sx = reinterpret_cast<float *>(xs);
    int8_t *zx = reinterpret_cast<int8_t *>(xs + 4);
    void *xpart = take(quantize_per_tensor_workspace((int64_t)mh));
    float *gate = reinterpret_cast<float *>(take(mi * 4));
    float *up = fused ? nullptr : reinterpret_cast<float *>(take(mi * 4));
    int8_t *qh = reinterpret_cast<int8_t *>(take(mi));
    char *hs = take(kAlign);
    float *sh = reinterpret_cast<float *>(hs);
    int8_t *zh = reinterpret_cast<int8_t *>(hs + 4);
    void *hpart = take(h_partials_bytes(d.m, d.inter));
    float *h = d.h ? d.h : gate;

    // Decode sizes (m = 1 at the LLaMA / Mistral widths): no quantize
    // launches.  The gate/up kernel quantizes x itself (every workgroup from
    // the min / max of all of x), and the down projection quantizes h from
    // gate/up's (min, max) partials of it: the same codes as the quantize
    // passes, two launches instead of five.
    if (fused && qlinear_qx_fits(d.m, d.inter, d.hidden, false) &&
        qlinear_qx_fits(d.m, d.hidden, d.inter, true) && aligned16(d.x) && aligned16(h)) {
        QSwigluDesc f;
        f.g.xf = d.x;
        f.g.m = d.m;
        f.g.n = d.inter;
        f.g.k = d.hidden;
        f.g.qw = d.qwg;
        f.g.sw = d.swg;
        f.g.w_rowsum = d.rsg;
        f.g.bias = d.bg;
        f.g.y = h;
        f.qw_up = d.qwu;
        f.sw_up = d.swu;
        f.rowsum_up = d.rsu;
        f.bias_up = d.bu;
        f.hpart = static_cast<float2 *>(hpart);
        int npart = 0;
        GFH_TRY(launch_qlinear_swiglu_i8(f, &npart, s));
        QLinearDesc q;
        q.xf = h;
        q.xpart = f.hpart;
        q.nxpart = npart;
        q.m = d.m;
        q.n = d.hidden;
        q.k = d.inter;
        q.qw = d.qwd;
        q.sw = d.swd;
        q.w_rowsum = d.rsd;
        q.bias = d.bd;
        q.y = d.y;
        return launch_qlinear_i8(q, s);
    }

    GFH_TRY(launch_quantize_per_tensor(d.x, (int64_t)mh, false, qx, sx, zx, xpart, s));
    QLinearDesc q;
    q.qx = qx;
    q.sx = sx;
    q.zx = zx;
    q.m = d.m;
    q.n = d.inter;
    q.k = d.hidden;
    q.qw = d.qwg;
    q.sw = d.swg;
    q.w_rowsum = d.rsg;
    q.bias = d.bg;
    if (fused) {
        QSwigluDesc f;
        f.g = q;
        f.g.y = h;
        f.qw_up = d.qwu;
        f.sw_up = d.swu;
        f.rowsum_up = d.rsu;
        f.bias_up = d.bu;
        f.hpart = static_cast<float2 *>(hpart);
        int npart = 0;
        GFH_TRY(launch_qlinear_swiglu_i8(f, &npart, s));
        GFH_TRY(launch_quantize_per_tensor_partials(h, (int64_t)mi, false, f.hpart, npart, qh, sh, zh, s));
    } else {
        q.y = gate;
        GFH_TRY(launch_qlinear_i8(q, s));
        q.qw = d.qwu;
        q.sw = d.swu;
        q.w_rowsum = d.rsu;
        q.bias = d.bu;
        q.y = up;
        GFH_TRY(launch_qlinear_i8(q, s));
        GFH_TRY(launch_silu_mul(gate, up, h, (int64_t)mi, s));
        GFH_TRY(launch_quantize_per_tensor(h, (int64_t)mi, false, qh, sh, zh, hpart, s));
    }
    q.qx = qh;
    q.sx = sh;
    q.zx = zh;
    q.n = d.hidden;
    q.k = d.inter;
    q.qw = d.qwd;
    q.sw = d.swd;
    q.w_rowsum = d.rsd;
    q.bias = d.bd;
    q.y = d.y;
    return launch_qlinear_i8(q, s);
}

}  // namespace gfh
