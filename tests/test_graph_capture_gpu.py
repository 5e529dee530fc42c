"""The decode path captured into a HIP graph (torch.cuda.CUDAGraph on a
dedicated stream) and replayed.  The library allocates its per-stream
buffers (split-K counters, zeroed by a fill kernel, and partial sums) on a
stream's first call, so every call runs once on the capture stream before
capture; the captured kernels then allocate nothing and record no memset.
Every replay must reproduce the eager outputs bit for bit (the kernels are
deterministic), with the outputs clobbered and other eager work run
between replays.  A call that would need a new buffer on a stream being
captured is refused before it issues any work."""
import numpy as np
import pytest

from _util import gemm_tol, to_dev

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _decode_setup(torch_dev):
    """One decode step: an int8 GEMV over a weight whose K is split over
    workgroups (arrival counters), an fp32 GEMV, and a MultiHeadAttention
    step over a KV cache (projections, KV attention with split keys,
    out_proj) with a caller workspace.  Outputs are preallocated."""
    import torch
    gh = _gh()
    from oracle import oracle as O
    b, k, n = 4, 4096, 2048 + 96
    x = to_dev(gh.normal((b, k), seed=31, tensor_id=0), torch_dev)
    wf = gh.normal((k, n), 0.0, 0.02, seed=31, tensor_id=1)
    qw, sc, zp = O.quantize_per_channel(wf, False)
    dqw, dsc, dzp, dwf = (to_dev(a, torch_dev) for a in (qw, sc, zp, wf))
    y8 = torch.empty((b, n), dtype=torch.float32, device=torch_dev)
    y32 = torch.empty((b, n), dtype=torch.float32, device=torch_dev)

    e, heads, past, cap = 512, 8, 300, 512
    q_in = to_dev(gh.normal((b, 1, e), seed=32, tensor_id=0), torch_dev)
    ws = [to_dev(gh.normal((e, e), 0.0, 0.04, seed=32, tensor_id=1 + i), torch_dev) for i in range(4)]
    bs = [to_dev(gh.normal((e,), 0.0, 0.1, seed=32, tensor_id=5 + i), torch_dev) for i in range(4)]
    kc = to_dev(gh.normal((b, cap, e), seed=32, tensor_id=9), torch_dev)
    vc = to_dev(gh.normal((b, cap, e), seed=32, tensor_id=10), torch_dev)
    mo = torch.empty((b, 1, e), dtype=torch.float32, device=torch_dev)
    mws = torch.empty(gh.ops.mha_workspace_size(b, 1, e) // 4 + 4, dtype=torch.float32, device=torch_dev)

    def step():
        gh.gemv_w8(x, dqw, dsc, dzp, out=y8)
        gh.gemv_f32(x, dwf, out=y32)
        gh.ops.mha_forward_cached(q_in, q_in, q_in, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], ws[3], bs[3],
                                  heads, kc, vc, past, out=mo, workspace=mws)

    return step, [y8, y32, mo, kc, vc]


def test_decode_step_graph_replays_match_eager(torch_dev):
    import torch
    step, outs = _decode_setup(torch_dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        step()  # first call on s: the per-stream buffers are allocated here
    s.synchronize()
    with torch.cuda.stream(s):
        step()
    s.synchronize()
    ref = [t.clone() for t in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.synchronize()
    for rep in range(4):
        for t in outs[:3]:
            t.fill_(float("nan"))
        step()  # eager calls on the default stream between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (t, r) in enumerate(zip(outs, ref)):
            assert torch.equal(t, r), (rep, i)


# torch warns that the graph is empty: nothing was captured, as intended.
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_capture_on_a_stream_without_its_buffers_is_refused(torch_dev):
    """An int8 GEMV with K split over workgroups on a stream that has never
    run it: its counters would have to be allocated (and zeroed) inside the
    capture, so the call fails with AllocationFailed before launching
    anything."""
    import torch
    gh = _gh()
    from ghostflow_hip import GhostFlowError
    from oracle import oracle as O
    b, k, n = 2, 4096, 2048 + 96
    x = to_dev(gh.normal((b, k), seed=33, tensor_id=0), torch_dev)
    qw, sc, zp = O.quantize_per_channel(gh.normal((k, n), 0.0, 0.02, seed=33, tensor_id=1), False)
    dqw, dsc, dzp = (to_dev(a, torch_dev) for a in (qw, sc, zp))
    y = torch.empty((b, n), dtype=torch.float32, device=torch_dev)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    raised = None
    with torch.cuda.graph(g, stream=s):
        try:
            gh.gemv_w8(x, dqw, dsc, dzp, out=y)
        except GhostFlowError as err:
            raised = err
    torch.cuda.synchronize()
    assert raised is not None and "captured" in str(raised)
    # The same call on that stream outside a capture allocates and works.
    with torch.cuda.stream(s):
        gh.gemv_w8(x, dqw, dsc, dzp, out=y)
    s.synchronize()
    xh = gh.normal((b, k), seed=33, tensor_id=0)
    wd = O.dequantize(qw, sc, zp)
    assert np.abs(y.cpu().numpy() - O.matmul(xh, wd)).max() <= gemm_tol(k, xh, wd)
