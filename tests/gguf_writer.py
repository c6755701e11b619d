"""Minimal GGUF writer for the reader tests (the published GGUF v2/v3 layout, little-endian).

A file is: magic "GGUF", u32 version, u64 tensor count, u64 metadata count; the metadata entries
(u64-length string key, u32 value type, value); the tensor table (name, u32 n_dims, u64 dims with the
innermost first, u32 ggml type, u64 offset into the data section); zero padding up to the alignment;
then the tensor data, each tensor placed at an aligned offset.  Knobs for the malformed-file tests
override single fields.
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292)}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def nbytes(ggml_type: int, shape) -> int:
    """Packed size of a tensor of `shape` ([outermost .. innermost])."""
    be, bb = BLOCK[ggml_type]
    n = 1
    for d in shape:
        n *= d
    assert n % be == 0
    return n // be * bb


def write(path, metadata, tensors, version=3, alignment=32, magic=b"GGUF", dims_override=None,
          type_override=None, offset_shift=0, truncate=None):
    """metadata: [(key, vtype, value)]; tensors: [(name, ggml_type, shape, data bytes)] with shape
    [outermost .. innermost] (a weight [out_dim, in_dim]).  Returns the data section's start."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    head += b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in metadata)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += len(data)
        off += (-off) % alignment
    for i, (name, gtype, shape, data) in enumerate(tensors):
        dims = list(reversed(shape)) if dims_override is None or i != 0 else dims_override
        t = gtype if type_override is None or i != 0 else type_override
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, offsets[i] + (offset_shift if i == 0 else 0))
    start = len(head) + (-len(head)) % alignment
    body = bytearray(head + b"\0" * (start - len(head)))
    for (_, _, _, data), o in zip(tensors, offsets):
        body += b"\0" * (start + o - len(body))
        body += data
    if truncate is not None:
        body = body[:truncate]
    with open(path, "wb") as f:
        f.write(bytes(body))
    return start
