"""CPU tests of the state dict file formats.

The oracle (oracle/ghostflw.py) restates the reference's writer and reader
(ghostflow-core/src/serialize.rs:20-196).  It is pinned here by a byte string
written out from the format's definition, by every error load_state_dict
raises, and by HashMap insert semantics.  The library's own parser
(gfh_state_dict_open / _entry / _find, host-only) is then checked against
the oracle on the same files: the same entries, the same rejections.
"""
import ctypes as C
import struct

import numpy as np
import pytest

from oracle import ghostflw as G


def test_known_answer_bytes():
    """{"w": [[1, 2], [3, 4]]} as save_state_dict writes it."""
    got = G.save_bytes([("w", np.array([[1, 2], [3, 4]], np.float32))])
    want = bytes.fromhex(
        "47484f5354464c57"      # "GHOSTFLW"
        "01000000"              # version 1
        "01000000"              # one tensor
        "01000000" "77"         # name length 1, "w"
        "02"                    # DType::F32
        "02000000"              # ndim 2
        "0200000000000000" "0200000000000000"
        "0000803f" "00000040" "00004040" "00008040")  # 1.0 2.0 3.0 4.0 little-endian
    assert got == want
    d = G.load_bytes(want)
    assert list(d) == ["w"] and d["w"][0] == 2
    np.testing.assert_array_equal(d["w"][1], [[1, 2], [3, 4]])


def test_dtype_byte_and_scalar_and_empty():
    buf = G.save_bytes([("s", np.float32(3.5), 7), ("e", np.zeros((0, 5), np.float32), 2)])
    d = G.load_bytes(buf)
    assert d["s"][0] == 7 and d["s"][1].shape == () and d["s"][1] == 3.5  # data is f32 whatever the byte says
    assert d["e"][1].shape == (0, 5)


def test_last_duplicate_wins():
    buf = G.save_bytes([("a", np.ones(2, np.float32)), ("b", np.zeros(1, np.float32)),
                        ("a", np.full(3, 7, np.float32))])
    d = G.load_bytes(buf)
    assert len(d) == 2
    np.testing.assert_array_equal(d["a"][1], [7, 7, 7])


def _bad_buffers():
    good = G.save_bytes([("w", np.arange(6, dtype=np.float32).reshape(2, 3))])
    yield "magic", b"GHOSTFLX" + good[8:], "Invalid file format"
    yield "version", good[:8] + struct.pack("<I", 2) + good[12:], "Unsupported version"
    dt = good.index(b"w") + 1
    yield "dtype", good[:dt] + b"\x0a" + good[dt + 1:], "Unknown dtype"
    yield "truncated data", good[:-1], "Read error"
    yield "truncated header", good[:10], "Read error"
    yield "count too large", good[:12] + struct.pack("<I", 2) + good[16:], "Read error"
    for label, raw in (("utf8", b"\xff"), ("overlong", b"\xc0\x80"), ("surrogate", b"\xed\xa0\x80"),
                       ("past 10ffff", b"\xf4\x90\x80\x80")):
        body = struct.pack("<I", len(raw)) + raw + b"\x02" + struct.pack("<I", 0) + struct.pack("<f", 1.0)
        yield label, b"GHOSTFLW" + struct.pack("<II", 1, 1) + body, "UTF-8"


@pytest.mark.parametrize("label,buf,msg", list(_bad_buffers()))
def test_oracle_rejects(label, buf, msg):
    with pytest.raises(G.FormatError, match=msg):
        G.load_bytes(buf)


def test_quantized_format_roundtrip():
    rng = np.random.default_rng(0)
    codes = rng.integers(-128, 128, size=(5, 7), dtype=np.int8)
    scales = rng.random(5).astype(np.float32)
    zps = rng.integers(-3, 4, size=5, dtype=np.int8)
    f = rng.standard_normal((3,)).astype(np.float32)
    buf = G.save_q_bytes([("q", "w", codes, scales, zps, 2), ("f", "b", f)])
    assert buf[:8] == b"GHOSTFLQ"
    d = G.load_bytes(buf)
    kind, scheme, c2, s2, z2 = d["w"]
    assert kind == "q" and scheme == 2
    np.testing.assert_array_equal(c2, codes)
    np.testing.assert_array_equal(s2, scales)
    np.testing.assert_array_equal(z2, zps)
    np.testing.assert_array_equal(d["b"][1], f)
    # payloads start at 64-byte file offsets
    assert buf.index(scales.tobytes()) % 64 == 0 and buf.index(codes.tobytes()) % 64 == 0
    assert buf.index(f.tobytes()) % 64 == 0


# ---- the library's parser against the oracle ---------------------------------

def _lib():
    from ghostflow_hip import _lib as L
    return L.load()


def _entries(path):
    L = _lib()
    h = C.c_void_p()
    rc = L.gfh_state_dict_open(str(path).encode(), C.byref(h))
    if rc != 0:
        return rc, L.gfh_last_error().decode(), None
    out = {}
    try:
        for i in range(L.gfh_state_dict_count(h)):
            name, kind, dtype, ndim, nsc = C.c_char_p(), C.c_int(), C.c_int(), C.c_int(), C.c_int64()
            dims = (C.c_int64 * 16)()
            assert L.gfh_state_dict_entry(h, i, C.byref(name), C.byref(kind), C.byref(dtype), C.byref(ndim), dims,
                                          16, C.byref(nsc)) == 0
            key = name.value.decode()
            out[key] = (kind.value, dtype.value, tuple(dims[d] for d in range(ndim.value)), nsc.value)
            assert L.gfh_state_dict_find(h, name.value) == i
        assert L.gfh_state_dict_find(h, b"no such name") == -1
        assert L.gfh_state_dict_entry(h, len(out), None, None, None, None, None, 0, None) == 1
    finally:
        L.gfh_state_dict_close(h)
    return 0, "", out


def test_library_parser_matches_oracle(tmp_path):
    rng = np.random.default_rng(1)
    ents = [("layer.0.weight", rng.standard_normal((4, 6)).astype(np.float32)),
            ("layer.0.bias", rng.standard_normal(4).astype(np.float32), 2),
            ("scalar", np.float32(1.25), 3), ("empty", np.zeros((2, 0, 3), np.float32)),
            ("layer.0.weight", rng.standard_normal((2, 2)).astype(np.float32)),
            ("ünïcödé", np.ones((1,), np.float32))]
    p = tmp_path / "m.gf"
    p.write_bytes(G.save_bytes(ents))
    rc, msg, got = _entries(p)
    assert rc == 0, msg
    ref = G.load_bytes(p.read_bytes())
    assert set(got) == set(ref)
    for k, (dtype, arr) in ref.items():
        assert got[k] == (0, dtype, arr.shape, 0), k
    # first appearance orders the entries, the last one supplies the data
    assert list(got) == ["layer.0.weight", "layer.0.bias", "scalar", "empty", "ünïcödé"]
    assert got["layer.0.weight"][2] == (2, 2)


@pytest.mark.parametrize("label,buf,msg", list(_bad_buffers()))
def test_library_rejects_what_the_reference_rejects(tmp_path, label, buf, msg):
    p = tmp_path / "bad.gf"
    p.write_bytes(buf)
    rc, err, _ = _entries(p)
    assert rc == 2, (label, rc)
    assert msg in err, (label, err)


def test_library_parses_quantized_format(tmp_path):
    codes = np.arange(12, dtype=np.int8).reshape(3, 4)
    p = tmp_path / "q.gfq"
    p.write_bytes(G.save_q_bytes([("q", "w", codes, np.ones(3, np.float32), np.zeros(3, np.int8)),
                                  ("q", "t", codes, np.ones(1, np.float32), np.zeros(1, np.int8), 1),
                                  ("f", "b", np.ones(4, np.float32), 2)]))
    rc, msg, got = _entries(p)
    assert rc == 0, msg
    assert got == {"w": (1, 0, (3, 4), 3), "t": (1, 1, (3, 4), 1), "b": (0, 2, (4,), 0)}
    # a scale count that is neither 1 nor dims[0] is rejected
    bad = G.save_q_bytes([("q", "w", codes, np.ones(3, np.float32), np.zeros(3, np.int8))])
    i = bad.index(struct.pack("<Q", 3) + b"\0")
    p.write_bytes(bad[:i] + struct.pack("<Q", 2) + bad[i + 8:])
    rc, msg, _ = _entries(p)
    assert rc == 2 and "scales" in msg


def test_library_open_errors(tmp_path):
    L = _lib()
    h = C.c_void_p()
    assert L.gfh_state_dict_open(str(tmp_path / "missing.gf").encode(), C.byref(h)) == 2
    assert b"Failed to open file" in L.gfh_last_error()
    assert L.gfh_state_dict_open(None, C.byref(h)) == 3
    (tmp_path / "empty.gf").write_bytes(b"")
    assert L.gfh_state_dict_open(str(tmp_path / "empty.gf").encode(), C.byref(h)) == 2
