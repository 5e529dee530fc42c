#!/usr/bin/env python3
"""bench.py -- throughput of GhostFlow's dense hot path on one MI355X.

Headline (the one JSON line on stdout): the fp32 Linear forward
y = x W^T + b at x [4096, 4096], W [4096, 4096], b [4096] -- the
configuration the headline metric is quoted on (Linear::forward,
ghostflow-nn/src/linear.rs:56-69, served by gfh_sgemm NT + bias).  One step
is one Linear forward over that batch, i.e. one sgemm kernel launch, with
every input already resident in HBM.

The same line carries
  * "roofline": the sgemm kernel's algorithmic FLOP per launch (2*M*N*K,
    bias excluded) over its average launch duration, timed with HIP events
    on the stream the kernel runs on, against the f32 MFMA peak;
  * "cpu_baseline": the reference CPU path (the oracle's restatement of
    Linear::forward -> data_f32 gather of W^T + matmul_blocked + broadcast
    bias add, single-threaded as the reference is) timed on this host on a
    bounded row sample and extrapolated to the full layer;
  * "components": the other hot-path kernels at their benchmark shapes
    (square fp32 GEMM, int8 linear, decode GEMV fp32 / int8, causal SDPA)
    and the decode path built on them (Linear at decode batch sizes,
    attention over a KV cache, one MultiHeadAttention decode step), each
    with its own roofline fraction.  These are supplementary numbers, not
    the headline.

Only 1 GPU is supported: --gpus N with N > 1 exits with an error.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ghost-flow_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "GEMM TFLOPS (fp32) / TOPS (int8) + decode GEMV GB/s, % roofline, 1×MI355X"
PEAK_F32 = 157.3e12   # dense f32 MFMA, FLOP/s
PEAK_I8 = 5.0e15      # dense i8 MFMA, OP/s
PEAK_HBM = 8.0e12     # HBM3E, B/s
MALL_BYTES = 256 << 20  # Infinity Cache; HBM-bound timings cycle > 2x this


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-components", action="store_true",
                    help="skip the supplementary per-kernel numbers")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-rows", type=int, default=768,
                    help="rows of x in the CPU-baseline sample (of 4096)")
    ap.add_argument("--only", default="",
                    help="comma list of components to run (sgemm,qlinear,gemv,sdpa,flash,softmax,quantize,"
                         "decode,swiglu,io); "
                         "used for focused profiling")
    ap.add_argument("--detail", default="", help="also write the full result JSON to this file")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy `steps` times (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    return ap.parse_args()


class Lib:
    """Direct ctypes calls into libghostflow_hip.so (no per-call Python checks)."""

    def __init__(self):
        import ghostflow_hip
        self.L = ghostflow_hip.lib()
        self.gh = ghostflow_hip

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: status {rc}: {self.L.gfh_last_error().decode()}")


# After any idle gap the GPU's clock needs ~25 ms of sustained work to reach
# its steady state (measured on this MI355X with back-to-back 4096^3 fp32
# GEMMs: 1140 us per launch right after 0.5 s idle, falling to 930 us after
# ~25 launches).  Every timing below therefore starts after at least
# SETTLE_S of back-to-back work.
SETTLE_S = 0.06


def settle(torch, fn, seconds=SETTLE_S):
    """Back-to-back calls of fn until `seconds` of wall time have passed."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    i = 0
    while True:
        for _ in range(4):
            fn(i)
            i += 1
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def event_time_ms(torch, fn, reps, warmup=3):
    """Average ms per call of fn() over `reps` back-to-back calls, timed
    with events on torch's current stream (the stream every call uses),
    after the clock has settled."""
    for _ in range(warmup):
        fn(0)
    settle(torch, fn)
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(reps):
        fn(i)
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


# ---------------------------------------------------------------------------
# headline: fp32 Linear 4096^3
# ---------------------------------------------------------------------------

def bench_linear(lib, torch, args):
    M = N = K = 4096
    g = lib.gh
    dev = torch.device("cuda:0")
    x = torch.from_numpy(g.normal((M, K), seed=0, tensor_id=0)).to(dev)
    w = torch.from_numpy(g.uniform((N, K), -1 / 64, 1 / 64, seed=0, tensor_id=1)).to(dev)
    b = torch.from_numpy(g.uniform((N,), -1 / 64, 1 / 64, seed=0, tensor_id=2)).to(dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    xp, wp, bp, yp = x.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr()

    def step():
        rc = L.gfh_sgemm(0, 1, M, N, K, 1.0, xp, K, wp, K, 0.0, yp, N, bp, stream)
        if rc:
            lib.check(rc, "gfh_sgemm")

    # Clock settle: ~60 ms of a separate 4096^3 GEMM on other buffers (the
    # GPU idled while the inputs were generated on the host), then the W
    # warmup steps and the K timed steps of the headline itself.
    sa = torch.randn((M, K), device=dev)
    sb = torch.randn((K, N), device=dev)
    sc = torch.empty((M, N), device=dev)
    settle(torch, lambda _: L.gfh_sgemm(0, 0, M, N, K, 1.0, sa.data_ptr(), K, sb.data_ptr(), N, 0.0,
                                        sc.data_ptr(), N, None, stream))
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = ev0.elapsed_time(ev1) / args.steps
    flops = 2.0 * M * N * K
    # sanity: one sampled output element against a float64 dot product
    xs = x[17].double().cpu()
    ws = w[1234].double().cpu()
    ref = float((xs * ws).sum() + b[1234].double().cpu())
    got = float(y[17, 1234].cpu())
    if abs(got - ref) > 1e-3:
        raise RuntimeError(f"linear sanity check failed: {got} vs {ref}")
    return {
        "wall_s": wall,
        "ms_per_step": wall * 1e3 / args.steps,
        "kernel_ms": ev_ms,
        "flops": flops,
        "value": flops / (wall / args.steps) / 1e12,
        "achieved": flops / (ev_ms * 1e-3) / 1e12,
    }


def cpu_baseline_linear(rows):
    """Reference CPU path of Linear::forward at [4096,4096]x[4096,4096]^T,
    timed on a row sample: the W^T gather (data_f32 of the t() view) is timed
    once in full, matmul_blocked and the bias add on `rows` rows of x, then
    scaled to 4096 rows (rows of the output are independent, identical work)."""
    import numpy as np
    from ghostflow_hip import synth
    from oracle import oracle as O
    M = N = K = 4096
    L = O.lib()
    x = synth.normal((rows, K), seed=0, tensor_id=0)
    w = synth.uniform((N, K), -1 / 64, 1 / 64, seed=0, tensor_id=1)
    b = synth.uniform((N,), -1 / 64, 1 / 64, seed=0, tensor_id=2)
    wt = np.empty((K, N), np.float32)
    t0 = time.perf_counter()
    L.gfo_transpose_last2(w, wt, 1, N, K)
    t_gather = time.perf_counter() - t0
    y = np.empty((rows, N), np.float32)
    t0 = time.perf_counter()
    L.gfo_matmul_blocked(x, wt, y, rows, K, N)
    t_mm = time.perf_counter() - t0
    t0 = time.perf_counter()
    L.gfo_add_row_bias(y, b, rows, N)
    t_bias = time.perf_counter() - t0
    scale = M / rows
    t_full = t_gather + (t_mm + t_bias) * scale
    return {
        "value": 2.0 * M * N * K / t_full / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle Linear::forward restatement (gather W^T in full {t_gather:.2f}s; "
                   f"matmul_blocked + bias on {rows}/4096 rows {t_mm + t_bias:.2f}s), "
                   f"extrapolated to 4096 rows: {t_full:.1f}s per forward"),
        "seconds_measured": t_gather + t_mm + t_bias,
    }


# ---------------------------------------------------------------------------
# the reference CPU path of each component (oracle restatement, this host)
# ---------------------------------------------------------------------------

class CpuRef:
    """Times the oracle's restatement of the reference CPU path (oracle/
    gf_oracle.c) for one component, threaded as the reference is: matmul,
    batched matmul, the view gather, quantize / dequantize and the mask on
    one thread (matmul.rs:101,147; quantization.rs:93,119; attention.rs:
    51-64), softmax and mul_scalar on a pool of nproc threads over rows
    (rayon's default pool: activation.rs:180-213, arithmetic.rs:69-72).

    Large workloads are timed on a bounded sample of independent rows or
    (b,h) slices -- identical work per row -- and scaled to the full shape
    ("extrapolated" in the sample text).  Tensor copies the reference makes
    (data_f32 of each operand, from_slice of the output) are memcpy's of the
    full tensors and are timed in full."""

    RATE = 14e9        # rough single-thread matmul_blocked FLOP/s, only to size samples
    TARGET_S = 0.4     # seconds of matmul per sample

    def __init__(self):
        import numpy as np
        from oracle import oracle as O
        self.np = np
        self.O = O
        self.L = O.lib()
        self.nproc = os.cpu_count() or 1
        self.rng = np.random.default_rng(0)
        self._warm()

    def _warm(self):
        """One small call of every primitive, so no sample pays first-use costs."""
        np, L = self.np, self.L
        self._copy_s(1 << 20)
        a = self._randn((8, 64))
        b = self._randn((64, 64))
        c = np.empty((8, 64), np.float32)
        L.gfo_matmul_blocked(a, b, c, 8, 64, 64)
        L.gfo_transpose_last2(b, np.empty((64, 64), np.float32), 1, 64, 64)
        q = np.empty(512, np.int8)
        s_, z_ = C.c_float(), C.c_int8()
        L.gfo_quantize_per_tensor(a.reshape(-1), 512, 0, q, C.byref(s_), C.byref(z_))
        d = np.empty(512, np.float32)
        L.gfo_dequantize(q, 8, 64, np.ones(8, np.float32), np.zeros(8, np.int8), 8, d)
        y = np.empty_like(a)
        self._par_rows(8, lambda r0, r1: L.gfo_softmax_lastdim(a.reshape(-1)[r0 * 64:r1 * 64],
                                                                y.reshape(-1)[r0 * 64:r1 * 64], r1 - r0, 64))

    # -- helpers ------------------------------------------------------------
    @staticmethod
    def _t(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    def _randn(self, shape):
        """N(0,1)-distributed f32 data: a 1 Mi-element random block repeated
        (the timed loops are data-independent; this only keeps the set-up of
        large operands fast)."""
        np = self.np
        n = int(np.prod(shape))
        if not hasattr(self, "_block"):
            self._block = self.rng.standard_normal(1 << 20, dtype=np.float32)
        reps = -(-n // self._block.size)
        return np.tile(self._block, reps)[:n].reshape(shape).copy() if reps > 1 else \
            self._block[:n].reshape(shape).copy()

    def _copy_s(self, nbytes):
        """One memcpy of nbytes (data_f32 / from_slice of a contiguous tensor)."""
        np = self.np
        src = np.ones(nbytes // 4, np.float32)
        dst = np.empty_like(src)
        dst[:1] = 0  # touch
        return self._t(lambda: np.copyto(dst, src))

    def _par_rows(self, rows, fn):
        """fn(r0, r1) over row chunks on nproc threads (rayon's pool)."""
        from concurrent.futures import ThreadPoolExecutor
        n = self.nproc
        step = max(1, -(-rows // (4 * n)))
        chunks = [(r, min(r + step, rows)) for r in range(0, rows, step)]
        with ThreadPoolExecutor(n) as pool:
            list(pool.map(lambda c: fn(*c), chunks))

    def _sample_rows(self, m, k, n):
        return int(max(1, min(m, round(self.TARGET_S * self.RATE / (2.0 * k * n)))))

    def matmul_s(self, m, k, n, b_transposed=False):
        """Tensor::matmul [m,k] x [k,n] (a W^T view when b_transposed, as
        Linear::forward): data_f32 of both operands (the W^T view is the
        gather), matmul_blocked, from_slice of the output.  Returns (seconds
        for the full shape, rows timed, seconds measured)."""
        np, L = self.np, self.L
        rows = self._sample_rows(m, k, n)
        a = self._randn((rows, k))
        t_copy = self._copy_s(4 * m * k) + self._copy_s(4 * m * n)
        if b_transposed:
            w = self._randn((n, k))
            bt = np.empty((k, n), np.float32)
            t_b = self._t(lambda: L.gfo_transpose_last2(w, bt, 1, n, k))
        else:
            bt = self._randn((k, n))
            t_b = self._copy_s(4 * k * n)
        c = np.empty((rows, n), np.float32)
        t_mm = self._t(lambda: L.gfo_matmul_blocked(a, bt, c, rows, k, n))
        full = t_copy + t_b + t_mm * (m / rows)
        return full, rows, t_copy + t_b + t_mm

    def result(self, value, unit, seconds_full, sample, cores=1, **extra):
        r = {"value": value, "unit": unit, "cores": cores, "kind": "port", "sample": sample,
             "seconds_full": seconds_full}
        r.update(extra)
        return r

    # -- components ---------------------------------------------------------
    def sgemm(self, n):
        full, rows, meas = self.matmul_s(n, n, n)
        fl = 2.0 * n ** 3
        ext = "extrapolated" if rows < n else "full"
        return self.result(fl / full / 1e12, "TFLOP/s", full,
                           f"oracle Tensor::matmul {n}^3 (2 operand copies + matmul_blocked + output copy); "
                           f"matmul_blocked on {rows}/{n} rows, {ext}: {full:.2f} s per call ({meas:.2f} s measured)")

    def matmul_backward(self, m, k, n):
        """matmul_backward's naive loops (backward.rs:131-160, restated by
        gfo_matmul_backward): grad_a rows and grad_b rows are independent, so
        each half is timed on a sample of its rows and scaled."""
        np, L = self.np, self.L
        ra, rb = min(m, 16), min(k, 4)  # (grad_b's loop reads a with stride k: ~0.2 s per row at 4096^2)
        g = self._randn((m, n))
        a = self._randn((m, k))
        b = self._randn((k, n))
        ga = np.empty((ra, k), np.float32)
        t_a = self._t(lambda: L.gfo_matmul_backward(g[:ra], a[:ra], b, ra, k, n, ga.ctypes.data, None))
        a_cols = np.ascontiguousarray(a[:, :rb])  # grad_b rows 0 .. rb-1 read these columns of a
        gb = np.empty((rb, n), np.float32)
        t_b = self._t(lambda: L.gfo_matmul_backward(g, a_cols, b[:rb], m, rb, n, None, gb.ctypes.data))
        full = t_a * (m / ra) + t_b * (k / rb)
        return self.result(4.0 * m * n * k / full / 1e12, "TFLOP/s", full,
                           f"oracle matmul_backward m={m} k={k} n={n}: grad_a on {ra}/{m} rows ({t_a:.2f} s), "
                           f"grad_b on {rb}/{k} rows ({t_b:.2f} s), extrapolated: {full:.1f} s per call")

    def batched_matmul(self, batch, m, k, n):
        """Tensor::matmul on [batch, m, k] @ [batch, k, n]: data_f32 of both
        operands, batched_matmul's i-j-k loop on a sample of slices, the
        output copy (the copies timed in full)."""
        np, L = self.np, self.L
        sl = min(batch, 4)
        a = self._randn((sl, m, k))
        b = self._randn((sl, k, n))
        c = np.empty((sl, m, n), np.float32)
        t_copy = self._copy_s(4 * batch * m * k) + self._copy_s(4 * batch * k * n) + self._copy_s(4 * batch * m * n)
        t_mm = self._t(lambda: L.gfo_batched_matmul(a.reshape(-1), sl, b.reshape(-1), sl, c.reshape(-1), sl, m, k, n))
        full = t_copy + t_mm * (batch / sl)
        return self.result(2.0 * batch * m * n * k / full / 1e12, "TFLOP/s", full,
                           f"oracle Tensor::matmul (batched_matmul) [{batch},{m},{k}] @ [{batch},{k},{n}]: operand and "
                           f"output copies in full, the loop on {sl}/{batch} slices ({t_mm:.2f} s), extrapolated: "
                           f"{full:.1f} s per call")

    def qlinear(self, m, n, k, per_tensor=True):
        """The reference's executable INT8 path: DynamicQuantization::
        quantize_activation (per tensor, asymmetric) of x, dequantize of x
        and get_weights (dequantize of W, per channel), then the fp32 layer
        x . W^T (gather + matmul_blocked).  Quantization is reported on its
        own (quantize_s) beside the dequantize and matmul parts."""
        np, L = self.np, self.L
        x = self._randn((m, k))
        qx = np.empty((m, k), np.int8)
        sx, zx = C.c_float(), C.c_int8()
        if per_tensor:
            t_q = self._t(lambda: L.gfo_quantize_per_tensor(x.reshape(-1), m * k, 0, qx.reshape(-1),
                                                             C.byref(sx), C.byref(zx)))
            sxa, zxa = np.array([sx.value], np.float32), np.array([zx.value], np.int8)
        else:
            sxa, zxa = np.empty(m, np.float32), np.empty(m, np.int8)
            t_q = self._t(lambda: L.gfo_quantize_per_channel(x.reshape(-1), m, k, 1, qx.reshape(-1), sxa, zxa))
        dx = np.empty((m, k), np.float32)
        t_dqx = self._t(lambda: L.gfo_dequantize(qx.reshape(-1), m, k, sxa, zxa, sxa.size, dx.reshape(-1)))
        qw = (self._randn((n, k)) * 40).astype(np.int8)
        sw = (self.rng.random(n, dtype=np.float32) * 1e-3).astype(np.float32)
        zw = np.zeros(n, np.int8)
        dw = np.empty((n, k), np.float32)
        t_dqw = self._t(lambda: L.gfo_dequantize(qw.reshape(-1), n, k, sw, zw, n, dw.reshape(-1)))
        del dw, qw
        t_lin, rows, _ = self.matmul_s(m, k, n, b_transposed=True)
        full = t_q + t_dqx + t_dqw + t_lin
        ops = 2.0 * m * n * k
        ext = "extrapolated" if rows < m else "full"
        return self.result(ops / full / 1e12, "TOP/s", full,
                           f"oracle quantize_activation + dequantize(x) + get_weights (dequantize W [{n},{k}]) + "
                           f"Linear x.W^T (gather + matmul_blocked on {rows}/{m} rows, {ext}); "
                           f"{full:.3f} s per call",
                           quantize_s=t_q, dequantize_s=t_dqx + t_dqw, matmul_s=t_lin)

    def gemv(self, bsz, int8, k=4096, n=14336):
        """Tensor::matmul x [B,K] . W [K,N] (int8: get_weights, i.e. dequantize
        of the [K,N] codes per K row, first), timed in full."""
        np, L = self.np, self.L
        t_deq = 0.0
        if int8:
            qw = (self._randn((k, n)) * 40).astype(np.int8)
            sw = (self.rng.random(k, dtype=np.float32) * 1e-3).astype(np.float32)
            zw = np.zeros(k, np.int8)
            w = np.empty((k, n), np.float32)
            t_deq = self._t(lambda: L.gfo_dequantize(qw.reshape(-1), k, n, sw, zw, k, w.reshape(-1)))
            del qw
        else:
            w = self._randn((k, n))
        x = self._randn((bsz, k))
        y = np.empty((bsz, n), np.float32)
        t_copy = self._copy_s(4 * k * n) + self._copy_s(4 * bsz * k) + self._copy_s(4 * bsz * n)
        t_mm = self._t(lambda: L.gfo_matmul_blocked(x, w, y, bsz, k, n))
        full = t_deq + t_copy + t_mm
        byts = k * n * (1 if int8 else 4) + 4 * bsz * k + 4 * bsz * n + (4 * k if int8 else 0)
        return self.result(byts / full / 1e9, "GB/s", full,
                           f"oracle {'get_weights (dequantize) + ' if int8 else ''}Tensor::matmul at M={bsz} "
                           f"(W copy + matmul_blocked + copies), full: {full * 1e3:.1f} ms per call",
                           matmul_s=t_mm, copy_s=t_copy, dequantize_s=t_deq)

    def sdpa(self, S, B=4, H=32, D=128, nslices=None):
        """scaled_dot_product_attention (attention.rs:11-49) with a causal
        [S,S] mask: K^T gather, batched QK^T, mul_scalar, the cycled mask,
        softmax, batched PV -- on a sample of (b,h) slices, extrapolated to
        B*H."""
        np, L = self.np, self.L
        bh = B * H
        ns = nslices or max(1, min(bh, int(round(self.TARGET_S * 3 * self.RATE / (4.0 * S * S * D)))))
        q, k, v = (self._randn((ns, S, D)) for _ in range(3))
        kt = np.empty((ns, D, S), np.float32)
        sc = np.empty((ns, S, S), np.float32)
        w = np.empty((ns, S, S), np.float32)
        o = np.empty((ns, S, D), np.float32)
        mask = np.tril(np.ones((S, S), np.float32)).reshape(-1)
        scale = np.float32(1.0) / np.sqrt(np.float32(D))
        t = {}
        t["gather"] = self._t(lambda: L.gfo_transpose_last2(k.reshape(-1), kt.reshape(-1), ns, S, D))
        t["qk"] = self._t(lambda: L.gfo_batched_matmul(q.reshape(-1), ns, kt.reshape(-1), ns, sc.reshape(-1),
                                                       ns, S, D, S))
        scf = sc.reshape(-1)
        rows = ns * S

        def scale_rows(r0, r1):
            seg = scf[r0 * S:r1 * S]
            L.gfo_mul_scalar(seg, seg.size, float(scale))
        t["mul_scalar"] = self._t(lambda: self._par_rows(rows, scale_rows))
        t["mask"] = self._t(lambda: L.gfo_apply_mask_cycled(scf, scf.size, mask, mask.size))
        wf = w.reshape(-1)

        def softmax_rows(r0, r1):
            xs = scf[r0 * S:r1 * S]
            ys = wf[r0 * S:r1 * S]
            L.gfo_softmax_lastdim(xs, ys, r1 - r0, S)
        t["softmax"] = self._t(lambda: self._par_rows(rows, softmax_rows))
        t["pv"] = self._t(lambda: L.gfo_batched_matmul(w.reshape(-1), ns, v.reshape(-1), ns, o.reshape(-1),
                                                       ns, S, S, D))
        meas = sum(t.values())
        full = meas * bh / ns
        fl = 4.0 * B * H * S * S * D * 0.5
        return self.result(fl / full / 1e12, "TFLOP/s", full,
                           f"oracle scaled_dot_product_attention with a causal [S,S] mask on {ns}/{bh} (b,h) "
                           f"slices ({meas:.2f} s), {'extrapolated' if ns < bh else 'full'}: {full:.1f} s per "
                           f"call; softmax and mul_scalar on {self.nproc} threads, the rest on one",
                           cores=self.nproc, stages_s={kk: round(vv * bh / ns, 4) for kk, vv in t.items()})

    def flash_attention(self, S, B=128, D=128):
        """FlashAttention::forward restated (the reference's loops, one
        thread) on a sample of batch entries -- independent, identical work
        -- extrapolated to B."""
        O = self.O
        nb = max(1, min(B, int(round(self.TARGET_S * self.RATE / (2.0 * S * S * D)))))
        q, k, v = (self._randn((nb, S, D)) for _ in range(3))
        scale = 1.0 / D ** 0.5
        meas = self._t(lambda: O.flash_attention_blockwise(q, k, v, 64, 64, True, scale))
        full = meas * B / nb
        fl = 4.0 * B * S * S * D * 0.5
        return self.result(fl / full / 1e12, "TFLOP/s", full,
                           f"oracle FlashAttention::forward (causal, 64 x 64 blocks) on {nb}/{B} batch entries "
                           f"({meas:.2f} s), {'extrapolated' if nb < B else 'full'}: {full:.1f} s per call")

    def softmax(self, rows, cols):
        np, L = self.np, self.L
        rs = min(rows, max(1, int(2e7 // cols)))
        x = self._randn((rs, cols))
        y = np.empty_like(x)
        xf, yf = x.reshape(-1), y.reshape(-1)

        def part(r0, r1):
            L.gfo_softmax_lastdim(xf[r0 * cols:r1 * cols], yf[r0 * cols:r1 * cols], r1 - r0, cols)
        meas = self._t(lambda: self._par_rows(rs, part))
        full = meas * rows / rs
        byts = 8.0 * rows * cols
        return self.result(byts / full / 1e9, "GB/s", full,
                           f"oracle softmax(-1) on {rs}/{rows} rows on {self.nproc} threads (rayon), "
                           f"{'extrapolated' if rs < rows else 'full'}: {full * 1e3:.1f} ms per call",
                           cores=self.nproc)

    def quantize(self, n):
        np, L = self.np, self.L
        x = self._randn((n,))
        q = np.empty(n, np.int8)
        s, z = C.c_float(), C.c_int8()
        full = self._t(lambda: L.gfo_quantize_per_tensor(x, n, 0, q, C.byref(s), C.byref(z)))
        return self.result(9.0 * n / full / 1e9, "GB/s", full,
                           f"oracle quantize_activation (per tensor, asymmetric) of {n} elements, full: "
                           f"{full * 1e3:.1f} ms per call")

    def kv_attention(self, B=4, H=32, D=128, kv_len=2048):
        """The attention step of MultiHeadAttention::forward_with_cache for
        one new token over kv_len - 1 cached positions (attention.rs:100-144):
        concat_tensors of the cached and new keys and of the values
        (:214-247), the head split of reshape_for_attention (:146-150) and
        scaled_dot_product_attention (:11-49), timed in full on one thread.
        Same algorithmic bytes as the GPU component (K, V, q, out)."""
        np, O = self.np, self.O
        E = H * D
        past_k, past_v = self._randn((B, kv_len - 1, E)), self._randn((B, kv_len - 1, E))
        k_new, v_new, q = self._randn((B, 1, E)), self._randn((B, 1, E)), self._randn((B, 1, E))

        def heads(t, n):  # [B, n, E] -> [B, H, n, D], one head at a time
            src = t.reshape(B, n, H, D)
            out = np.empty((B, H, n, D), np.float32)
            for hh in range(H):
                out[:, hh] = src[:, :, hh, :]
            return out

        def step():
            kc = np.concatenate([past_k, k_new], axis=1)
            vc = np.concatenate([past_v, v_new], axis=1)
            O.sdpa(heads(q, 1), heads(kc, kv_len), heads(vc, kv_len))
        step()
        full = self._t(step)
        byts = 2 * 4 * B * kv_len * E + 8 * B * E
        return self.result(byts / full / 1e9, "GB/s", full,
                           f"oracle concat_tensors (K, V) + reshape_for_attention + scaled_dot_product_attention "
                           f"over {kv_len} positions, B={B}, {H} heads of {D}, full: {full * 1e3:.1f} ms per step")

    def mha_decode(self, B=4, H=32, D=128, past=2047):
        """One decode step of MultiHeadAttention::forward_with_cache
        (attention.rs:100-144): the q / k / v projections (Linear::forward,
        W^T gather + matmul_blocked + bias), the cache concatenation, SDPA
        and out_proj, through the oracle's composite, timed in full."""
        np, O = self.np, self.O
        E = H * D
        w = [self._randn((E, E)) * np.float32(1 / 64) for _ in range(4)]
        bias = [self._randn((E,)) * np.float32(1 / 64) for _ in range(4)]
        x = self._randn((B, 1, E))
        pk, pv = self._randn((B, past, E)), self._randn((B, past, E))

        def step():
            O.mha_forward_with_cache(x, x, x, w[0], bias[0], w[1], bias[1], w[2], bias[2], w[3], bias[3], H,
                                     past_key=pk, past_value=pv)
        full = self._t(step)
        byts = 4 * 4 * E * E + 2 * 4 * B * (past + 1) * E + 4 * B * E * 6
        return self.result(byts / full / 1e9, "GB/s", full,
                           f"oracle MultiHeadAttention::forward_with_cache, B={B}, 1 new token, {past} cached "
                           f"positions, E={E}, {H} heads (4 Linear + concat + SDPA), full: "
                           f"{full * 1e3:.1f} ms per step", tokens_per_s=B / full)

    def state_dict_load(self, path):
        """load_state_dict + read_tensor (serialize.rs:48-88,124-167) of a
        file already in the page cache, restated byte for byte
        (oracle/ghostflw.py): the file read and the little-endian decode of
        every tensor into host memory, timed in full on one thread."""
        from oracle import ghostflw
        nbytes = os.path.getsize(path)

        def load():
            with open(path, "rb") as fh:
                ghostflw.load_bytes(fh.read())
        load()
        full = min(self._t(load) for _ in range(3))
        return self.result(nbytes / full / 1e9, "GB/s", full,
                           f"oracle GHOSTFLW/GHOSTFLQ reader (read + decode into host memory) of a {nbytes / 1e6:.0f} "
                           f"MB file from the page cache, full, best of 3: {full * 1e3:.1f} ms")

    def linear(self, m, n, k):
        full, rows, meas = self.matmul_s(m, k, n, b_transposed=True)
        t_bias = self._copy_s(4 * m * n)  # the broadcast add writes a new [m, n] tensor (same traffic)
        full += t_bias
        return full, rows

    def swiglu(self, m, int8, H=4096, I=11008):
        """SwiGLU::forward: gate, up, down Linear layers (int8: each through
        the reference's quantize_activation + dequantize + get_weights +
        fp32 Linear path) and silu(gate) * up."""
        np, L = self.np, self.L
        parts = []
        for n_out, n_in in ((I, H), (I, H), (H, I)):
            if int8:
                parts.append(self.qlinear(m, n_out, n_in)["seconds_full"])
            else:
                parts.append(self.linear(m, n_out, n_in)[0])
        g = self._randn((min(m, 256), I))
        u = self._randn((min(m, 256), I))
        h = np.empty_like(g)
        t_silu = self._t(lambda: L.gfo_silu_mul(g.reshape(-1), u.reshape(-1), h.reshape(-1), g.size)) * m / g.shape[0]
        full = sum(parts) + t_silu
        ops = 6.0 * m * H * I
        return self.result(ops / full / 1e12, "TOP/s" if int8 else "TFLOP/s", full,
                           f"oracle SwiGLU::forward ({'int8 composite per Linear' if int8 else 'fp32 Linear'} "
                           f"x3 + silu*up, matmuls on row samples, extrapolated): {full:.3f} s per call")


def host_record(torch):
    """The machine the bench ran on: host CPU, memory, ROCm / torch, GPU."""
    rec = {"nproc": os.cpu_count()}
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    rec["cpu_model"] = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        with open("/proc/meminfo") as fh:
            for ln in fh:
                if ln.startswith("MemTotal:"):
                    rec["ram_gib"] = round(int(ln.split()[1]) / 2 ** 20, 1)
                    break
    except OSError:
        pass
    try:
        with open("/opt/rocm/.info/version") as fh:
            rec["rocm"] = fh.read().strip()
    except OSError:
        pass
    rec["torch"] = torch.__version__
    try:
        p = torch.cuda.get_device_properties(0)
        rec["gpu"] = f"{p.name} ({getattr(p, 'gcnArchName', '')}, {p.multi_processor_count} CUs, " \
                     f"{p.total_memory / 2 ** 30:.0f} GiB)"
    except Exception:  # noqa: BLE001
        pass
    import subprocess
    for cmd in (["amd-smi", "metric", "--clock"], ["rocm-smi", "--showclocks"]):
        try:
            out = subprocess.run(cmd, capture_output=True, text=True, timeout=20)
        except (OSError, subprocess.SubprocessError):
            continue
        if out.returncode == 0 and out.stdout.strip():
            lines = [ln.strip() for ln in out.stdout.splitlines() if ln.strip() and "=" not in ln[:3]]
            rec["clocks_after_run"] = " | ".join(lines[:24])[:1200]
            rec["clocks_cmd"] = " ".join(cmd)
            break
    return rec


# ---------------------------------------------------------------------------
# supplementary components
# ---------------------------------------------------------------------------

def comp_sgemm(lib, torch, n):
    dev = torch.device("cuda:0")
    a = torch.randn((n, n), device=dev)
    b = torch.randn((n, n), device=dev)
    c = torch.empty((n, n), device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    ap, bp, cp = a.data_ptr(), b.data_ptr(), c.data_ptr()

    def f(_):
        L.gfh_sgemm(0, 0, n, n, n, 1.0, ap, n, bp, n, 0.0, cp, n, None, s)
    reps = int(min(200, max(5, 1.0 / (2.0 * n ** 3 / 50e12))))  # about 1 s of GPU time
    ms = event_time_ms(torch, f, reps)
    fl = 2.0 * n ** 3
    return {"name": f"sgemm_nn_{n}", "ms": ms, "value": fl / ms / 1e9, "unit": "TFLOP/s",
            "frac": fl / ms / 1e9 / (PEAK_F32 / 1e12), "bound": "mfma_f32"}


def comp_matmul_backward(lib, torch, m, k, n):
    """matmul_backward (ghostflow-autograd/src/backward.rs:131-160) of C = a @ b,
    a [m, k], b [k, n]: grad_a = grad . b^T (NT) and grad_b = a^T . grad
    (transposed A), one gfh_matmul_backward_f32 call, 2 x 2mnk FLOP."""
    dev = torch.device("cuda:0")
    g = torch.randn((m, n), device=dev)
    a = torch.randn((m, k), device=dev)
    b = torch.randn((k, n), device=dev)
    ga = torch.empty((m, k), device=dev)
    gb = torch.empty((k, n), device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    gp, ap, bp, gap, gbp = g.data_ptr(), a.data_ptr(), b.data_ptr(), ga.data_ptr(), gb.data_ptr()

    def f(_):
        L.gfh_matmul_backward_f32(gp, ap, bp, m, k, n, gap, gbp, s)
    fl = 4.0 * m * n * k
    reps = int(min(100, max(5, 1.0 / (fl / 50e12))))
    ms = event_time_ms(torch, f, reps)
    return {"name": f"matmul_backward_m{m}_k{k}_n{n}", "ms": ms, "value": fl / ms / 1e9, "unit": "TFLOP/s",
            "frac": fl / ms / 1e9 / (PEAK_F32 / 1e12), "bound": "mfma_f32"}


def comp_batched_matmul(lib, torch, batch, m, k, n):
    """Tensor::matmul on 3-D operands (batched_matmul, matmul.rs:122-170):
    [batch, m, k] @ [batch, k, n], the attention-score shape, through
    gfh_sgemm_strided_batched."""
    dev = torch.device("cuda:0")
    a = torch.randn((batch, m, k), device=dev)
    b = torch.randn((batch, k, n), device=dev)
    c = torch.empty((batch, m, n), device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    ap, bp, cp = a.data_ptr(), b.data_ptr(), c.data_ptr()

    def f(_):
        L.gfh_sgemm_strided_batched(0, 0, m, n, k, 1.0, ap, k, m * k, batch, bp, n, k * n, batch, 0.0, cp, n, m * n,
                                    batch, None, s)
    fl = 2.0 * batch * m * n * k
    reps = int(min(200, max(5, 1.0 / (fl / 50e12))))
    ms = event_time_ms(torch, f, reps)
    return {"name": f"batched_matmul_b{batch}_m{m}_k{k}_n{n}", "ms": ms, "value": fl / ms / 1e9,
            "unit": "TFLOP/s", "frac": fl / ms / 1e9 / (PEAK_F32 / 1e12), "bound": "mfma_f32"}


def comp_qlinear(lib, torch, m, n, k, per_tensor=True):
    """Config 3: W ~ N(0, 0.02) quantized per channel (symmetric), x ~ N(0, 1)
    quantized per tensor (asymmetric), as DynamicQuantization does, with this
    library's own quantize kernels (torch only draws the normal samples)."""
    dev = torch.device("cuda:0")
    gh = lib.gh
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn((m, k), device=dev, generator=g)
    if per_tensor:
        qx, sx, zx = gh.quantize_per_tensor(x, symmetric=False)
    else:
        qx, sx, zx = gh.quantize_per_channel(x, symmetric=True)
    del x
    # rotate weight copies when the working set would sit in the MALL
    wbytes = n * k
    ncopy = max(1, min(16, -(-2 * MALL_BYTES // wbytes))) if m <= 256 else 1
    qws = []
    for _ in range(ncopy):
        w = torch.randn((n, k), device=dev, generator=g) * 0.02
        qw, sw, _zw = gh.quantize_per_channel(w, symmetric=True)
        qws.append(qw)
        del w
    rs = [gh.qweight_rowsum(q) for q in qws]
    y = torch.empty((m, n), device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    ptrs = [(q.data_ptr(), r.data_ptr()) for q, r in zip(qws, rs)]

    def f(i):
        qp, rp = ptrs[i % ncopy]
        L.gfh_qlinear_i8(qx.data_ptr(), sx.data_ptr(), zx.data_ptr(), 0 if per_tensor else 1, qp,
                         sw.data_ptr(), rp, None, y.data_ptr(), None, m, n, k, s)
    ops = 2.0 * m * n * k
    reps = 200 if ops < 5e10 else 100
    ms = event_time_ms(torch, f, reps)
    byts = m * k + n * k + 4 * m * n + 8 * n
    tops = ops / ms / 1e9
    gbs = byts / ms / 1e6
    attain = min(PEAK_I8, ops / byts * PEAK_HBM)
    return {"name": f"qlinear_i8_m{m}_n{n}_k{k}", "ms": ms, "value": tops, "unit": "TOP/s",
            "gbps": gbs, "frac": ops / (ms * 1e-3) / attain,
            "bound": "mfma_i8" if attain == PEAK_I8 else "hbm", "weight_copies": ncopy}


def comp_qlinear_dynamic(lib, torch, m, n, k):
    """The INT8 linear on fp32 activations (gfh_qlinear_dynamic_i8):
    DynamicQuantization's quantize_activation of x (per tensor, asymmetric)
    and the INT8 linear in one call -- one launch at m <= 4, where
    qlinear_i8_* above times the linear alone on codes quantized beforehand.
    Same data as comp_qlinear; algorithmic bytes count x in fp32."""
    dev = torch.device("cuda:0")
    gh = lib.gh
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn((m, k), device=dev, generator=g)
    wbytes = n * k
    ncopy = max(1, min(16, -(-2 * MALL_BYTES // wbytes)))
    qws, sw = [], None
    for _ in range(ncopy):
        w = torch.randn((n, k), device=dev, generator=g) * 0.02
        qw, sw, _zw = gh.quantize_per_channel(w, symmetric=True)
        qws.append(qw)
        del w
    rs = [gh.qweight_rowsum(q) for q in qws]
    y = torch.empty((m, n), device=dev)
    nws = int(lib.L.gfh_qlinear_dynamic_i8_workspace_size(m, k))
    ws = torch.empty((nws + 3) // 4, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    ptrs = [(q.data_ptr(), r.data_ptr()) for q, r in zip(qws, rs)]

    def f(i):
        qp, rp = ptrs[i % ncopy]
        L.gfh_qlinear_dynamic_i8(x.data_ptr(), qp, sw.data_ptr(), rp, None, y.data_ptr(), m, n, k,
                                 ws.data_ptr(), ws.numel() * 4, s)
    ms = event_time_ms(torch, f, 200)
    ops = 2.0 * m * n * k
    byts = 4 * m * k + n * k + 4 * m * n + 8 * n
    gbs = byts / ms / 1e6
    attain = min(PEAK_I8, ops / byts * PEAK_HBM)
    return {"name": f"qlinear_dynamic_i8_m{m}_n{n}_k{k}", "ms": ms, "value": ops / ms / 1e9, "unit": "TOP/s",
            "gbps": gbs, "frac": ops / (ms * 1e-3) / attain,
            "bound": "mfma_i8" if attain == PEAK_I8 else "hbm", "weight_copies": ncopy}


def comp_gemv(lib, torch, bsz, int8):
    dev = torch.device("cuda:0")
    K, N = 4096, 14336
    wbytes = K * N * (1 if int8 else 4)
    ncopy = max(3, -(-2 * MALL_BYTES // wbytes) + 1)
    x = torch.randn((bsz, K), device=dev)
    y = torch.empty((bsz, N), device=dev)
    if int8:
        ws = [torch.randint(-127, 128, (K, N), dtype=torch.int8, device=dev) for _ in range(ncopy)]
        sc = torch.rand((K,), device=dev) * 1e-3
    else:
        ws = [torch.randn((K, N), device=dev) * 0.02 for _ in range(ncopy)]
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    wp = [t.data_ptr() for t in ws]
    if int8:
        def f(i):
            L.gfh_gemv_w8(x.data_ptr(), wp[i % ncopy], sc.data_ptr(), None, y.data_ptr(), bsz, K, N, s)
    else:
        def f(i):
            L.gfh_gemv_f32(x.data_ptr(), wp[i % ncopy], y.data_ptr(), bsz, K, N, s)
    ms = event_time_ms(torch, f, 300)
    byts = wbytes + 4 * bsz * K + 4 * bsz * N + (4 * K if int8 else 0)
    gbs = byts / ms / 1e6
    del ws
    return {"name": f"gemv_{'w8' if int8 else 'f32'}_b{bsz}", "ms": ms, "value": gbs, "unit": "GB/s",
            "frac": gbs * 1e9 / PEAK_HBM, "bound": "hbm", "weight_copies": ncopy}


def comp_sdpa(lib, torch, S):
    dev = torch.device("cuda:0")
    B, H, D = 4, 32, 128
    q = torch.randn((B, H, S, D), device=dev)
    k = torch.randn((B, H, S, D), device=dev)
    v = torch.randn((B, H, S, D), device=dev)
    o = torch.empty_like(q)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    scale = float(1.0 / (128.0 ** 0.5))

    def f(_):
        L.gfh_sdpa_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), None, B, H, S, S, D,
                       scale, 1, None, 0, s)
    ms = event_time_ms(torch, f, 50 if S <= 512 else 10)
    fl = 4.0 * B * H * S * S * D * 0.5
    return {"name": f"sdpa_causal_b4_h32_s{S}_d128", "ms": ms, "value": fl / ms / 1e9, "unit": "TFLOP/s",
            "frac": fl / ms / 1e9 / (PEAK_F32 / 1e12), "bound": "mfma_f32"}


def comp_flash_attention(lib, torch, S, B=128, D=128):
    """FlashAttention::forward (ghostflow-nn/src/flash_attention.rs:81-250)
    on [B, S, D] with FlashAttentionConfig::causal(1/sqrt(D)) and the
    default 64 x 64 blocks (gfh_flash_attention_f32, single-pass form) --
    config 5's (b,h) slices as the layer's batch.  Work: 4*B*S^2*D * 1/2
    FLOP (causal, the FlashAttention convention, as for SDPA); the bound is
    the f32 MFMA peak."""
    dev = torch.device("cuda:0")
    q = torch.randn((B, S, D), device=dev)
    k = torch.randn((B, S, D), device=dev)
    v = torch.randn((B, S, D), device=dev)
    o = torch.empty_like(q)
    L = lib.L
    wsb = int(L.gfh_flash_attention_workspace_size(B, S, S))
    ws = torch.empty((wsb + 3) // 4, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    scale = float(1.0 / (D ** 0.5))

    def f(_):
        L.gfh_flash_attention_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, S, S, D, 64, 64, 1,
                                  scale, ws.data_ptr(), wsb, s)
    ms = event_time_ms(torch, f, 50 if S <= 512 else 10)
    fl = 4.0 * B * S * S * D * 0.5
    return {"name": f"flash_attention_causal_b{B}_s{S}_d{D}_blocks64", "ms": ms, "value": fl / ms / 1e9,
            "unit": "TFLOP/s", "frac": fl / ms / 1e9 / (PEAK_F32 / 1e12), "bound": "mfma_f32"}


def comp_linear_decode(lib, torch, m):
    """Linear::forward at decode batch sizes: x [m, 4096] . W^T + b with W
    [4096, 4096] (gfh_sgemm NT -> the row-dot GEMV up to 4 rows, the skinny
    f32-MFMA kernel up to 64).  HBM-bound below m ~ 40: bytes = 4*N*K +
    4*m*K + 4*N (bias) + 4*m*N; the roofline is min(f32 MFMA, AI * HBM)."""
    dev = torch.device("cuda:0")
    N = K = 4096
    wbytes = 4 * N * K
    ncopy = max(3, -(-2 * MALL_BYTES // wbytes) + 1)
    ws = [torch.empty((N, K), device=dev).uniform_(-1 / 64, 1 / 64) for _ in range(ncopy)]
    x = torch.randn((m, K), device=dev)
    bias = torch.empty((N,), device=dev).uniform_(-1 / 64, 1 / 64)
    y = torch.empty((m, N), device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    wp = [t.data_ptr() for t in ws]

    def f(i):
        L.gfh_sgemm(0, 1, m, N, K, 1.0, x.data_ptr(), K, wp[i % ncopy], K, 0.0, y.data_ptr(), N,
                    bias.data_ptr(), s)
    ms = event_time_ms(torch, f, 300)
    byts = wbytes + 4 * m * K + 4 * N + 4 * m * N
    gbs = byts / ms / 1e6
    fl = 2.0 * m * N * K
    attain = min(PEAK_F32, fl / byts * PEAK_HBM)
    del ws
    return {"name": f"linear_decode_m{m}_4096", "ms": ms, "value": gbs, "unit": "GB/s",
            "tflops": fl / ms / 1e9, "frac": fl / (ms * 1e-3) / attain,
            "bound": "mfma_f32" if attain == PEAK_F32 else "hbm", "weight_copies": ncopy}


def _kv_sets(torch, dev, B, C, E, n):
    return [(torch.randn((B, C, E), device=dev), torch.randn((B, C, E), device=dev)) for _ in range(n)]


def comp_kv_attention(lib, torch, B=4, H=32, D=128, kv_len=2048):
    """One decode step of attention over a [B, kv_len, E] cache
    (gfh_kv_attention_f32, Sq = 1).  HBM-bound: bytes = 2*4*B*kv_len*E
    (K and V) + 8*B*E (q, out)."""
    dev = torch.device("cuda:0")
    E = H * D
    kvbytes = 2 * 4 * B * kv_len * E
    ncopy = max(2, -(-2 * MALL_BYTES // kvbytes) + 1)
    sets = _kv_sets(torch, dev, B, kv_len, E, ncopy)
    q = torch.randn((B, 1, E), device=dev)
    o = torch.empty_like(q)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    ptrs = [(k.data_ptr(), v.data_ptr()) for k, v in sets]
    scale = float(1.0 / (D ** 0.5))

    def f(i):
        kp, vp = ptrs[i % ncopy]
        L.gfh_kv_attention_f32(q.data_ptr(), E, kp, vp, kv_len, E, o.data_ptr(), E, None, B, H, 1, kv_len, D,
                               scale, 0, None, 0, s)
    ms = event_time_ms(torch, f, 200)
    byts = kvbytes + 8 * B * E
    gbs = byts / ms / 1e6
    del sets
    return {"name": f"kv_attention_b{B}_h{H}_d{D}_kv{kv_len}", "ms": ms, "value": gbs, "unit": "GB/s",
            "frac": gbs * 1e9 / PEAK_HBM, "bound": "hbm", "cache_copies": ncopy}


def comp_mha_decode(lib, torch, B=4, H=32, D=128, past=2047):
    """One decode step of MultiHeadAttention::forward_with_cache: 1 new
    token per sequence, E = 4096, 32 heads, `past` cached positions
    (gfh_mha_forward_with_cache_f32: 4 projections + cache attention).
    HBM-bound: bytes = 4 * 4*E*E (weights) + 2*4*B*(past+1)*E (cache) plus
    the small activations."""
    dev = torch.device("cuda:0")
    E = H * D
    C = past + 1
    per_set = 4 * 4 * E * E + 2 * 4 * B * C * E
    ncopy = max(2, -(-2 * MALL_BYTES // per_set) + 1)
    sets = []
    for _ in range(ncopy):
        w = [torch.empty((E, E), device=dev).uniform_(-1 / 64, 1 / 64) for _ in range(4)]
        kc, vc = _kv_sets(torch, dev, B, C, E, 1)[0]
        sets.append((w, kc, vc))
    bias = [torch.empty((E,), device=dev).uniform_(-1 / 64, 1 / 64) for _ in range(4)]
    x = torch.randn((B, 1, E), device=dev)
    out = torch.empty_like(x)
    ws = torch.empty((int(lib.L.gfh_mha_workspace_size(B, 1, E)) + 3) // 4, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L
    bp = [t.data_ptr() for t in bias]
    ptrs = [([t.data_ptr() for t in w], kc.data_ptr(), vc.data_ptr()) for w, kc, vc in sets]

    def step(i, stream):
        wp, kp, vp = ptrs[i % ncopy]
        L.gfh_mha_forward_with_cache_f32(x.data_ptr(), x.data_ptr(), x.data_ptr(), wp[0], bp[0], wp[1], bp[1],
                                         wp[2], bp[2], wp[3], bp[3], kp, vp, C, past, None, 0, 0,
                                         out.data_ptr(), None, B, 1, 1, E, H, ws.data_ptr(),
                                         ws.numel() * 4, stream)

    ms = event_time_ms(torch, lambda i: step(i, s), 100)
    # The same step captured once per weight/cache set into a HIP graph and
    # replayed (a serving loop's form: one launch per step).  Each stream
    # gets its split-K buffers on its first call, so the capture stream runs
    # every set once before capture.
    byts = per_set + 4 * B * E * 6
    gbs = byts / ms / 1e6
    graph = {"graph_ms": None}
    try:
        cap = torch.cuda.Stream()
        with torch.cuda.stream(cap):
            for i in range(ncopy):
                step(i, cap.cuda_stream)
        cap.synchronize()
        graphs = []
        for i in range(ncopy):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                step(i, cap.cuda_stream)
            graphs.append(g)
        torch.cuda.synchronize()
        gms = event_time_ms(torch, lambda i: graphs[i % ncopy].replay(), 100)
        graph = {"graph_ms": gms, "graph_tokens_per_s": B / (gms * 1e-3),
                 "graph_frac": byts / gms / 1e6 * 1e9 / PEAK_HBM}
        del graphs
    except Exception as err:  # a side measurement: the step's own figure above stands
        torch.cuda.synchronize()
        graph["graph_error"] = str(err)[:200]
    del sets
    return {"name": f"mha_decode_step_b{B}_e{E}_h{H}_past{past}", "ms": ms, "value": gbs, "unit": "GB/s",
            "tokens_per_s": B / (ms * 1e-3), "frac": gbs * 1e9 / PEAK_HBM, "bound": "hbm",
            "set_copies": ncopy, **graph}


def comp_swiglu(lib, torch, m, int8, H=4096, I=11008):
    """SwiGLU::forward (llama.rs:276-286) at the LLaMA-7B feed-forward shape,
    hidden 4096, intermediate 11008, x [m, 4096] ~ N(0, 1).
    * int8 (gfh_swiglu_i8): W ~ N(0, 0.02) per-channel symmetric codes; x
      and h quantized per tensor on the device; gate/up as one fused launch.
    * fp32 (gfh_swiglu_f32): W ~ U(+-sqrt(6/in)), b ~ U(+-1/sqrt(in)).
    Work: 6*m*H*I ops (three GEMMs).  Algorithmic bytes: the three weights
    (s_w*3*H*I) + x + y (8*m*H); the bound is min(MFMA peak, AI * HBM)."""
    dev = torch.device("cuda:0")
    gh = lib.gh
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    sw = 1 if int8 else 4
    wbytes = 3 * H * I * sw
    ncopy = max(1, -(-2 * MALL_BYTES // wbytes) + 1) if m <= 256 else 1
    sets = []
    for _ in range(ncopy):
        layer = []
        for n_out, n_in in ((I, H), (I, H), (H, I)):
            if int8:
                w = torch.randn((n_out, n_in), device=dev, generator=g) * 0.02
                q, sc, _ = gh.quantize_per_channel(w, symmetric=True)
                del w
                b = (torch.rand((n_out,), device=dev, generator=g) * 2 - 1) / n_in ** 0.5
                layer.append((q, sc, gh.qweight_rowsum(q), b))
            else:
                w = (torch.rand((n_out, n_in), device=dev, generator=g) * 2 - 1) * (6.0 / n_in) ** 0.5
                b = (torch.rand((n_out,), device=dev, generator=g) * 2 - 1) / n_in ** 0.5
                layer.append((w, b))
        sets.append(layer)
    x = torch.randn((m, H), device=dev, generator=g)
    y = torch.empty((m, H), device=dev)
    L = lib.L
    nws = int(L.gfh_swiglu_i8_workspace_size(m, H, I) if int8 else L.gfh_swiglu_f32_workspace_size(m, I))
    ws = torch.empty((nws + 3) // 4, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    ptrs = [[t.data_ptr() for part in layer for t in part] for layer in sets]

    def f(i):
        p = ptrs[i % ncopy]
        if int8:
            L.gfh_swiglu_i8(x.data_ptr(), m, H, I, *p, y.data_ptr(), None, ws.data_ptr(), nws, s)
        else:
            L.gfh_swiglu_f32(x.data_ptr(), m, H, I, *p, y.data_ptr(), None, ws.data_ptr(), nws, s)
    ops = 6.0 * m * H * I
    ms = event_time_ms(torch, f, 20 if ops > 1e12 else 100)
    byts = wbytes + 8 * m * H
    peak = PEAK_I8 if int8 else PEAK_F32
    attain = min(peak, ops / byts * PEAK_HBM)
    del sets
    return {"name": f"swiglu_{'i8' if int8 else 'f32'}_m{m}_h{H}_i{I}", "ms": ms,
            "value": ops / ms / 1e9, "unit": "TOP/s" if int8 else "TFLOP/s", "gbps": byts / ms / 1e6,
            "frac": ops / (ms * 1e-3) / attain,
            "bound": ("mfma_i8" if int8 else "mfma_f32") if attain == peak else "hbm", "weight_sets": ncopy}


def comp_state_dict_load(lib, torch, int8, cpu=None):
    """Weight load, file -> HBM: the three LLaMA-7B MLP weights (4096 x 11008
    each) as a GHOSTFLW state dict (fp32, 541 MB) or a GHOSTFLQ file of their
    int8 codes + scales (135 MB), read from the page cache through
    gfh_state_dict_read_* (mapped file, pinned double-buffered H2D copies).
    Bound: the host link (PCIe 5 x16, ~64 GB/s per direction)."""
    import tempfile
    dev = torch.device("cuda:0")
    gh = lib.gh
    H, I = 4096, 11008
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    state = {}
    for name, shape in (("mlp.gate_proj.weight", (I, H)), ("mlp.up_proj.weight", (I, H)),
                        ("mlp.down_proj.weight", (H, I))):
        w = torch.randn(shape, device=dev, generator=g) * 0.02
        state[name] = gh.quantize_per_channel(w, symmetric=True) if int8 else w
    fd, path = tempfile.mkstemp(suffix=".gfq" if int8 else ".gf", dir=os.environ.get("TMPDIR", "/tmp"))
    os.close(fd)
    try:
        gh.save_state_dict(path, state, quantized_format=int8)
        nbytes = os.path.getsize(path)
        with gh.StateDict(path) as sd:
            keys = sd.keys()
            outs = {k: (tuple(torch.empty_like(t) for t in state[k]) if int8 else torch.empty_like(state[k]))
                    for k in keys}

            def load_all():
                for k in keys:
                    i = sd._info[k][0]
                    o = outs[k]
                    if int8:
                        lib.check(lib.L.gfh_state_dict_read_q8(sd._h, i, o[0].data_ptr(), o[1].data_ptr(),
                                                               o[2].data_ptr(), None), "read_q8")
                    else:
                        lib.check(lib.L.gfh_state_dict_read_f32(sd._h, i, o.data_ptr(), None), "read_f32")
            load_all()  # warm the page cache and the staging buffers
            torch.cuda.synchronize()
            reps = 5
            t0 = time.perf_counter()
            for _ in range(reps):
                load_all()
            torch.cuda.synchronize()
            sec = (time.perf_counter() - t0) / reps
        for k in keys:
            a, b = (state[k], outs[k]) if not int8 else (state[k][0], outs[k][0])
            if not torch.equal(a, b):
                raise RuntimeError(f"state dict reload mismatch in {k}")
        cpu_res = None
        if cpu is not None:  # the reference's reader on the same file, while it exists
            try:
                cpu_res = cpu.state_dict_load(path)
            except Exception as e:  # noqa: BLE001
                cpu_res = {"error": str(e)}
    finally:
        os.unlink(path)
    gbs = nbytes / sec / 1e9
    r = {"name": f"state_dict_load_{'ghostflq_i8' if int8 else 'ghostflw_f32'}_llama7b_mlp", "ms": sec * 1e3,
         "value": gbs, "unit": "GB/s", "bytes": nbytes, "frac": gbs / 64.0, "bound": "pcie5_x16"}
    if cpu_res is not None:
        r["cpu_baseline"] = cpu_res
    return r


def comp_quantize(lib, torch, m, k=4096):
    """DynamicQuantization::quantize_activation on the device
    (gfh_quantize_i8_per_tensor, asymmetric) of x [m, k] ~ N(0, 1): a min/max
    pass, then the codes.  Algorithmic bytes = 9 per element (two reads of
    the f32 input -- the codes need the global min/max first -- and one
    int8 write).  HBM-bound."""
    dev = torch.device("cuda:0")
    n = m * k
    ncopy = max(1, -(-2 * MALL_BYTES // (4 * n)) + 1)
    xs = [torch.randn((n,), device=dev) for _ in range(ncopy)]
    q = torch.empty((n,), dtype=torch.int8, device=dev)
    sc = torch.empty((1,), device=dev)
    zp = torch.empty((1,), dtype=torch.int8, device=dev)
    L = lib.L
    wsb = int(L.gfh_quantize_i8_per_tensor_workspace_size(n))
    ws = torch.empty((wsb + 3) // 4, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    xp = [t.data_ptr() for t in xs]

    def f(i):
        L.gfh_quantize_i8_per_tensor(xp[i % ncopy], n, 0, q.data_ptr(), sc.data_ptr(), zp.data_ptr(),
                                     ws.data_ptr(), wsb, s)
    ms = event_time_ms(torch, f, 200)
    byts = 9.0 * n
    gbs = byts / ms / 1e6
    del xs
    return {"name": f"quantize_per_tensor_m{m}_k{k}", "ms": ms, "value": gbs, "unit": "GB/s",
            "frac": gbs * 1e9 / PEAK_HBM, "bound": "hbm", "input_copies": ncopy}


def comp_softmax(lib, torch, S, B=4, H=32):
    """Tensor::softmax(-1) over the SDPA score shape [B*H*S, S]
    (gfh_softmax_lastdim_f32).  Algorithmic bytes = 8 per element (read x,
    write y).  HBM-bound."""
    dev = torch.device("cuda:0")
    rows = B * H * S
    x = torch.randn((rows, S), device=dev) * 3
    y = torch.empty_like(x)
    s = torch.cuda.current_stream(dev).cuda_stream
    L = lib.L

    def f(_):
        L.gfh_softmax_lastdim_f32(x.data_ptr(), y.data_ptr(), rows, S, s)
    ms = event_time_ms(torch, f, 100 if S <= 512 else 20)
    byts = 8.0 * rows * S
    gbs = byts / ms / 1e6
    return {"name": f"softmax_rows{rows}_cols{S}", "ms": ms, "value": gbs, "unit": "GB/s",
            "frac": gbs * 1e9 / PEAK_HBM, "bound": "hbm"}


def run_components(lib, torch, only, cpu=None):
    """Every component's GPU figure, each with the reference CPU path's
    figure for the same workload (`cpu_baseline`) when `cpu` is given.  The
    square fp32 GEMMs run last among the GPU figures (the headline Linear
    settles the clock again itself).

    The CPU baselines run after every GPU figure is taken: numpy's BLAS
    threads keep spinning on the host cores for a while after a call, and
    the components whose calls take a few microseconds on the GPU are bound
    by how fast the host submits them (the per-tensor quantize of a [256,
    4096] activation measured 24.9 us per call right after a CPU baseline,
    7.5 us without one)."""
    want = set(filter(None, only.split(","))) or {"sgemm", "qlinear", "gemv", "sdpa", "flash", "softmax",
                                                  "quantize", "decode", "swiglu", "io", "backward"}
    out = []
    pending = []  # (record, cpu_fn): CPU baselines, run after the GPU figures

    def add(fn, *a, cpu_fn=None, **kw):
        try:
            r = fn(lib, torch, *a, **kw)
        except Exception as e:  # report, keep going
            r = {"name": fn.__name__ + repr(a), "error": str(e)}
        torch.cuda.empty_cache()
        if cpu is not None and cpu_fn is not None and "error" not in r:
            pending.append((r, cpu_fn))
        log("  " + json.dumps(r))
        out.append(r)

    def cpu_baselines():
        if pending:
            log("bench: CPU baselines of the components")
        for r, cpu_fn in pending:
            try:
                r["cpu_baseline"] = cpu_fn()
            except Exception as e:  # noqa: BLE001
                r["cpu_baseline"] = {"error": str(e)}
            log("  " + json.dumps({"name": r["name"], "cpu_baseline": r["cpu_baseline"]}))

    if "io" in want:
        for int8 in (False, True):
            add(comp_state_dict_load, int8, cpu=cpu)
    if "qlinear" in want:
        add(comp_qlinear, 4096, 4096, 4096, cpu_fn=lambda: cpu.qlinear(4096, 4096, 4096))
        for m in (1, 16, 256, 4096):
            add(comp_qlinear, m, 11008, 4096, cpu_fn=lambda m=m: cpu.qlinear(m, 11008, 4096))
        for m in (1, 4):
            add(comp_qlinear_dynamic, m, 11008, 4096, cpu_fn=lambda m=m: cpu.qlinear(m, 11008, 4096))
    if "quantize" in want:
        for m in (256, 4096):
            add(comp_quantize, m, cpu_fn=lambda m=m: cpu.quantize(m * 4096))
    if "gemv" in want:
        for int8 in (False, True):
            for bsz in (1, 4, 8):
                add(comp_gemv, bsz, int8, cpu_fn=lambda b=bsz, i=int8: cpu.gemv(b, i))
    if "sdpa" in want:
        for S in (512, 2048):
            add(comp_sdpa, S, cpu_fn=lambda S=S: cpu.sdpa(S))
    if "flash" in want:
        for S in (512, 2048):
            add(comp_flash_attention, S, cpu_fn=lambda S=S: cpu.flash_attention(S))
    if "softmax" in want:
        for S in (512, 2048):
            add(comp_softmax, S, cpu_fn=lambda S=S: cpu.softmax(4 * 32 * S, S))
    if "decode" in want:
        for m in (1, 4, 8, 16, 64):
            add(comp_linear_decode, m, cpu_fn=lambda m=m: _cpu_linear_result(cpu, m, 4096, 4096))
        add(comp_kv_attention, cpu_fn=lambda: cpu.kv_attention())
        add(comp_mha_decode, cpu_fn=lambda: cpu.mha_decode())
    if "swiglu" in want:
        for m in (1, 16, 256, 4096):
            add(comp_swiglu, m, True, cpu_fn=lambda m=m: cpu.swiglu(m, True))
        for m in (1, 16, 4096):
            add(comp_swiglu, m, False, cpu_fn=lambda m=m: cpu.swiglu(m, False))
        # Mistral-7B's feed-forward width (ghostflow-ml/src/deep/architectures/transformer.rs:2021)
        for m in (1, 16, 256, 4096):
            add(comp_swiglu, m, True, I=14336, cpu_fn=lambda m=m: cpu.swiglu(m, True, I=14336))
        for m in (1, 16):
            add(comp_swiglu, m, False, I=14336, cpu_fn=lambda m=m: cpu.swiglu(m, False, I=14336))
    if "backward" in want:
        add(comp_matmul_backward, 4096, 4096, 4096, cpu_fn=lambda: cpu.matmul_backward(4096, 4096, 4096))
        add(comp_batched_matmul, 128, 512, 128, 512, cpu_fn=lambda: cpu.batched_matmul(128, 512, 128, 512))
    if "sgemm" in want:
        for n in (1024, 2048, 4096, 8192):
            add(comp_sgemm, n, cpu_fn=lambda n=n: cpu.sgemm(n))
    cpu_baselines()
    return out


def _cpu_linear_result(cpu, m, n, k):
    full, rows = cpu.linear(m, n, k)
    byts = 4.0 * n * k + 4 * m * k + 4 * n + 4 * m * n
    return cpu.result(byts / full / 1e9, "GB/s", full,
                      f"oracle Linear::forward at m={m} (W^T gather + matmul_blocked on {rows}/{m} rows + bias), "
                      f"{'extrapolated' if rows < m else 'full'}: {full * 1e3:.1f} ms per call")


def calib_copy(torch, steps):
    """A plain copy of 1 GiB: reads 2^30 bytes and writes 2^30 bytes per
    launch, so its FETCH_SIZE / WRITE_SIZE per dispatch give the counters'
    scale factors."""
    dev = torch.device("cuda:0")
    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes_read": nbytes, "calib_copy_bytes_written": nbytes,
                      "launches": steps}), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.calib_copy:
        calib_copy(torch, args.steps)
        return
    lib = Lib()
    lib.check(lib.L.gfh_init(), "gfh_init")
    # The timed loops call the C ABI back to back; the per-call pointer
    # validation (hipPointerGetAttributes / hipMemGetAddressRange) is host
    # work that a serving loop with known-good buffers switches off.
    lib.L.gfh_set_pointer_checks(0)

    components = []
    if not args.no_components:
        log("bench: components" + ("" if args.no_cpu else " (each with the reference CPU path timed on this host)"))
        components = run_components(lib, torch, args.only, None if args.no_cpu else CpuRef())

    log(f"bench: fp32 Linear 4096^3, warmup {args.warmup}, steps {args.steps}")
    h = bench_linear(lib, torch, args)
    log(f"bench: {h['ms_per_step']:.3f} ms/step, {h['value']:.2f} TFLOP/s "
        f"(kernel {h['kernel_ms']:.3f} ms, {h['achieved']:.2f} TFLOP/s)")

    cpu = None
    if not args.no_cpu:
        log(f"bench: CPU baseline on {args.cpu_rows} rows")
        cpu = cpu_baseline_linear(args.cpu_rows)
        log(f"bench: CPU {cpu['value'] * 1e3:.3f} GFLOP/s ({cpu['sample']})")

    # HBM bytes per launch of the Linear kernel, measured with rocprofv3
    # FETCH_SIZE / WRITE_SIZE and scaled by a plain copy of known size; the
    # summary (with its commands) lives beside the other profiles.
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "sgemm_linear4096_traffic.md")
    if os.path.exists(tfile):
        with open(tfile) as fh:
            for ln in fh:
                if ln.startswith("bytes_per_launch:"):
                    traffic = int(ln.split(":", 1)[1])

    host = host_record(torch)
    detail_path = args.detail or os.path.join(ROOT, "gpurun_out", "bench_detail.json")
    line = headline_line(args.steps, args.warmup, h, cpu, traffic, host, components,
                         os.path.relpath(detail_path, ROOT))
    detail = dict(line)
    detail["host"] = host
    detail["components"] = [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in c.items()}
                            for c in components]
    try:
        os.makedirs(os.path.dirname(detail_path), exist_ok=True)
        with open(detail_path, "w") as fh:
            json.dump(detail, fh, indent=1)
    except OSError as e:
        log(f"bench: could not write {detail_path}: {e}")
    print(json.dumps(line), flush=True)


# Components whose fraction of roofline the north star sets a target for:
# fp32 GEMM >= 0.60 of f32 MFMA at 4096^3, INT8 >= 0.50 of i8 MFMA at
# 4096^3, decode GEMV >= 0.70 of HBM at B = 1/4/8.
NORTH_STAR_COMPONENTS = {
    "sgemm_nn_4096": 0.60,
    "qlinear_i8_m4096_n4096_k4096": 0.50,
    "gemv_f32_b1": 0.70, "gemv_f32_b4": 0.70, "gemv_f32_b8": 0.70,
    "gemv_w8_b1": 0.70, "gemv_w8_b4": 0.70, "gemv_w8_b8": 0.70,
}
# The result line must stay well inside what a log tail keeps.
LINE_LIMIT = 2048


def headline_line(steps, warmup, h, cpu, traffic, host, components, detail_rel):
    """The one stdout JSON line: the headline and its roofline and CPU
    baseline, the host in brief, and for the north star's target components
    only [microseconds, fraction of roofline, target].  Every component with
    its own CPU baseline goes to stderr and to the detail file instead."""
    ns = {}
    for c in components:
        t = NORTH_STAR_COMPONENTS.get(c.get("name"))
        if t is not None and "ms" in c:
            ns[c["name"]] = [round(c["ms"] * 1e3, 1), round(c.get("frac", 0.0), 3), t]
    line = {
        "metric": METRIC,
        "value": round(h["value"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(h["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (counter-based seed-0 generator: x ~ N(0,1), W, b ~ U(-1/64, 1/64))",
        "config": {"workload": "fp32 Linear forward y = x W^T + b (Linear::forward via gfh_sgemm NT+bias)",
                   "m": 4096, "k": 4096, "n": 4096, "bias": True, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(h["achieved"], 3), "peak": PEAK_F32 / 1e12,
                     "unit": "TFLOP/s", "frac": round(h["achieved"] / (PEAK_F32 / 1e12), 4),
                     "traffic": traffic},
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "host": {k: host[k] for k in ("nproc", "cpu_model", "ram_gib", "rocm", "gpu") if k in host},
        "north_star": ns,
        "components": {"count": len(components), "file": detail_rel},
    }
    if len(json.dumps(line)) > LINE_LIMIT:
        # the sample text is the only free-form field of any length
        line["cpu_baseline"]["sample"] = line["cpu_baseline"]["sample"][:240]
    return line


if __name__ == "__main__":
    main()
