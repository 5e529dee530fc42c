"""Byte-level restatement of GhostFlow's state dict files -- TEST
INFRASTRUCTURE ONLY (the checker of the library's reader and writer; only
tests/ and bench.py's cpu_baseline leg use it).

GHOSTFLW follows ghostflow-core/src/serialize.rs:
  save_state_dict  :20-45   magic, u32 version 1, u32 count, entries
  load_state_dict  :48-88   magic check, version <= 1, count, entries into a
                            HashMap (a repeated name keeps its last tensor)
  write_tensor     :90-122  u32 name length, name, u8 dtype, u32 ndim,
                            u64 dims, numel x f32 (data_f32, little-endian)
  read_tensor      :124-167 the same, String::from_utf8 on the name,
                            byte_to_dtype (0-9, else an error), f32 data
  dtype bytes      :169-196 F16 0, BF16 1, F32 2, F64 3, I8 4, I16 5, I32 6,
                            I64 7, U8 8, Bool 9
GHOSTFLQ is this library's own file for QuantizedTensor
(ghostflow-nn/src/quantization.rs:40-51); its layout is the one
include/ghostflow_hip.h specifies.  Everything is little-endian.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC_W = b"GHOSTFLW"
MAGIC_Q = b"GHOSTFLQ"
VERSION = 1
DTYPES = {"F16": 0, "BF16": 1, "F32": 2, "F64": 3, "I8": 4, "I16": 5, "I32": 6, "I64": 7, "U8": 8, "Bool": 9}
ALIGN = 64


class FormatError(ValueError):
    """The reference's GhostError::InvalidOperation on a bad file."""


def write_tensor(name: str, data, dtype: int = 2) -> bytes:
    """serialize.rs:90-122."""
    a = np.array(data, dtype="<f4", order="C")  # keeps 0-d tensors 0-d
    nb = name.encode("utf-8")
    out = [struct.pack("<I", len(nb)), nb, struct.pack("<B", dtype), struct.pack("<I", a.ndim)]
    out += [struct.pack("<Q", d) for d in a.shape]
    out.append(a.tobytes())
    return b"".join(out)


def save_bytes(entries) -> bytes:
    """save_state_dict (serialize.rs:20-45) over (name, array[, dtype])
    entries in the given order (the reference iterates its HashMap)."""
    parts = [MAGIC_W, struct.pack("<I", VERSION), struct.pack("<I", len(entries))]
    for e in entries:
        parts.append(write_tensor(*e))
    return b"".join(parts)


class _Reader:
    def __init__(self, buf: bytes):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        if n < 0 or self.pos + n > len(self.buf):
            raise FormatError("Read error")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def u8(self):
        return self.take(1)[0]

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def align(self, a: int):
        nxt = -(-self.pos // a) * a
        if nxt > len(self.buf):
            raise FormatError("Read error")
        self.pos = nxt


def _name(r: _Reader) -> str:
    n = r.u32()
    try:
        return r.take(n).decode("utf-8", errors="strict")
    except UnicodeDecodeError as e:
        raise FormatError("Invalid UTF-8") from e


def load_bytes(buf: bytes) -> dict:
    """load_state_dict (serialize.rs:48-88) and read_tensor (:124-167);
    returns name -> (dtype byte, float32 array of the stored shape).  For a
    GHOSTFLQ buffer kind-1 entries map to ("q", scheme, codes, scales,
    zero_points)."""
    r = _Reader(buf)
    magic = r.take(8)
    if magic not in (MAGIC_W, MAGIC_Q):
        raise FormatError("Invalid file format")
    quant = magic == MAGIC_Q
    version = r.u32()
    if version > VERSION:
        raise FormatError(f"Unsupported version: {version} (max: {VERSION})")
    count = r.u32()
    out = {}
    for _ in range(count):
        name = _name(r)
        kind = r.u8() if quant else 0
        if kind > 1:
            raise FormatError(f"unknown entry kind {kind}")
        dtype = r.u8()
        if kind == 0 and dtype > 9:
            raise FormatError(f"Unknown dtype: {dtype}")
        if kind == 1 and dtype > 2:
            raise FormatError(f"unknown quantization scheme {dtype}")
        ndim = r.u32()
        dims = tuple(r.u64() for _ in range(ndim))
        numel = int(np.prod(dims, dtype=object)) if dims else 1
        if kind == 0:
            if quant:
                r.align(ALIGN)
            data = np.frombuffer(r.take(numel * 4), dtype="<f4").astype(np.float32).reshape(dims)
            out[name] = (dtype, data)  # HashMap insert: a later entry replaces an earlier one
            continue
        nscales = r.u64()
        if nscales != 1 and (ndim == 0 or nscales != dims[0] or numel == 0):
            raise FormatError("bad scale count")
        r.align(ALIGN)
        scales = np.frombuffer(r.take(nscales * 4), dtype="<f4").astype(np.float32)
        zps = np.frombuffer(r.take(nscales), dtype=np.int8).copy()
        r.align(ALIGN)
        codes = np.frombuffer(r.take(numel), dtype=np.int8).reshape(dims).copy()
        out[name] = ("q", dtype, codes, scales, zps)
    return out


def save_q_bytes(entries) -> bytes:
    """GHOSTFLQ over entries ("f", name, array[, dtype]) and
    ("q", name, codes, scales, zero_points[, scheme])."""
    parts = [MAGIC_Q, struct.pack("<I", VERSION), struct.pack("<I", len(entries))]
    pos = sum(len(p) for p in parts)

    def add(b):
        nonlocal pos
        parts.append(b)
        pos += len(b)

    def pad():
        add(b"\0" * ((-pos) % ALIGN))

    for e in entries:
        nb = e[1].encode("utf-8")
        add(struct.pack("<I", len(nb)) + nb)
        if e[0] == "f":
            a = np.array(e[2], dtype="<f4", order="C")
            add(struct.pack("<BBI", 0, e[3] if len(e) > 3 else 2, a.ndim))
            add(b"".join(struct.pack("<Q", d) for d in a.shape))
            pad()
            add(a.tobytes())
        else:
            codes = np.ascontiguousarray(e[2], dtype=np.int8)
            scales = np.ascontiguousarray(np.atleast_1d(e[3]), dtype="<f4")
            zps = np.ascontiguousarray(np.atleast_1d(e[4]), dtype=np.int8)
            add(struct.pack("<BBI", 1, e[5] if len(e) > 5 else 0, codes.ndim))
            add(b"".join(struct.pack("<Q", d) for d in codes.shape))
            add(struct.pack("<Q", scales.size))
            pad()
            add(scales.tobytes())
            add(zps.tobytes())
            pad()
            add(codes.tobytes())
    return b"".join(parts)
