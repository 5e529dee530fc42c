"""State dict files to and from HBM (gfh_state_dict_*), checked against the
oracle's restatement of the reference's writer and reader
(ghostflow-core/src/serialize.rs:20-196):
* a file the reference would write loads to the device bit for bit,
  including tensors larger than one staging chunk, scalars and empty ones;
* a file the library writes from device memory is byte-identical to the
  reference's output for the same tensors in the same order;
* GHOSTFLQ round-trips QuantizedTensor codes, scales and zero points, and
  the reloaded weights give the INT8 linear bit-identical outputs."""
import numpy as np
import pytest

from oracle import ghostflw as G
from oracle import oracle as O
from _util import to_dev, to_np

pytestmark = pytest.mark.gpu


def _gh():
    import ghostflow_hip
    return ghostflow_hip


def _tensors(rng):
    return [("embed", rng.standard_normal((4096, 1100)).astype(np.float32)),   # 18 MB: two staging chunks
            ("layer.0.weight", rng.standard_normal((48, 64)).astype(np.float32)),
            ("layer.0.bias", rng.standard_normal(48).astype(np.float32)),
            ("scale", np.float32(0.5)), ("empty", np.zeros((3, 0), np.float32)),
            ("nan_inf", np.array([np.nan, np.inf, -np.inf, -0.0], np.float32))]


def test_load_reference_file(torch_dev, tmp_path):
    rng = np.random.default_rng(0)
    ents = _tensors(rng)
    p = tmp_path / "model.gf"
    p.write_bytes(G.save_bytes(ents))
    got = _gh().load_state_dict(p, device=torch_dev)
    assert list(got) == [n for n, _ in ents]
    for name, arr in ents:
        t = got[name]
        assert tuple(t.shape) == np.shape(arr), name
        np.testing.assert_array_equal(to_np(t).view(np.uint32), np.asarray(arr, np.float32).view(np.uint32))


def test_save_is_byte_identical_to_reference(torch_dev, tmp_path):
    rng = np.random.default_rng(1)
    ents = _tensors(rng)
    import torch
    # torch.from_numpy keeps the 0-d scalar 0-d (np.ascontiguousarray would not)
    state = {n: torch.from_numpy(np.array(a, np.float32)).to(torch_dev) for n, a in ents}
    p = tmp_path / "saved.gf"
    _gh().save_state_dict(p, state, dtypes={"scale": 3})
    want = G.save_bytes([(n, a, 3 if n == "scale" else 2) for n, a in ents])
    assert p.read_bytes() == want


def test_quantized_roundtrip_and_linear(torch_dev, tmp_path):
    gh = _gh()
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((1000, 512)) * 0.02).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    codes, scales, zps = gh.quantize_per_channel(to_dev(w, torch_dev), symmetric=True)
    p = tmp_path / "q.gfq"
    gh.save_state_dict(p, {"fc.weight": (codes, scales, zps), "fc.bias": to_dev(b, torch_dev)},
                       quantized_format=True)
    # the oracle reads what the library wrote
    ref = G.load_bytes(p.read_bytes())
    kind, scheme, c2, s2, z2 = ref["fc.weight"]
    assert kind == "q" and scheme == 0
    np.testing.assert_array_equal(c2, to_np(codes))
    np.testing.assert_array_equal(s2.view(np.uint32), to_np(scales).view(np.uint32))
    np.testing.assert_array_equal(z2, to_np(zps))
    np.testing.assert_array_equal(ref["fc.bias"][1], b)
    # and the library reads it back to the device
    with gh.StateDict(p) as sd:
        assert sd.info("fc.weight") == (1, 0, (1000, 512), 1000)
        c3, s3, z3 = sd.tensor("fc.weight", torch_dev)
        b3 = sd.tensor("fc.bias", torch_dev)
    assert bool((c3 == codes).all()) and bool((s3 == scales).all()) and bool((z3 == zps).all())
    # the reloaded weights drive the INT8 linear to the same bits
    x = rng.standard_normal((16, 512)).astype(np.float32)
    qx, sx, zx = gh.quantize_per_tensor(to_dev(x, torch_dev), symmetric=False)
    y1, _ = gh.qlinear(qx, sx, zx, codes, scales, bias=to_dev(b, torch_dev))
    y2, _ = gh.qlinear(qx, sx, zx, c3, s3, bias=b3)
    assert bool((y1 == y2).all())
    yo, _ = O.qlinear_i8(to_np(qx), to_np(sx), to_np(zx), False, c2, s2, b, want_acc=False)
    np.testing.assert_array_equal(to_np(y2), yo)


def test_read_errors(torch_dev, tmp_path):
    """An entry read as the other kind is refused before any copy; so is a
    quantized entry in a GHOSTFLW file."""
    import torch
    from ghostflow_hip.ops import _check
    gh = _gh()
    p = tmp_path / "m.gf"
    p.write_bytes(G.save_bytes([("w", np.ones((4, 4), np.float32))]))
    buf = torch.empty(64, dtype=torch.int8, device=torch_dev)
    with gh.StateDict(p) as sd:
        with pytest.raises(gh.GhostFlowError, match="read_f32"):
            _check(gh.lib().gfh_state_dict_read_q8(sd._h, 0, buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), None))
    q = tmp_path / "q.gfq"
    q.write_bytes(G.save_q_bytes([("q", "w", np.zeros((2, 4), np.int8), np.ones(2, np.float32),
                                   np.zeros(2, np.int8))]))
    out = torch.empty(8, device=torch_dev)
    with gh.StateDict(q) as sd:
        with pytest.raises(gh.GhostFlowError, match="read_q8"):
            _check(gh.lib().gfh_state_dict_read_f32(sd._h, 0, out.data_ptr(), None))
    with pytest.raises(gh.GhostFlowError, match="quantized_format"):
        gh.save_state_dict(tmp_path / "x.gf", {"q": (torch.zeros(2, 2, dtype=torch.int8, device=torch_dev),
                                                     torch.ones(2, device=torch_dev),
                                                     torch.zeros(2, dtype=torch.int8, device=torch_dev))})
