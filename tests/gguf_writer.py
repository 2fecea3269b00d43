"""A minimal GGUF writer for the tests: synthetic model files in the layout
the reference's parser reads (src/gguf/gguf_parser.cpp:144-345): header,
metadata key/values, tensor infos, then the tensor data region at the next
multiple of the alignment, each tensor at an aligned offset within it.

Tensors given as (name, dims, type, data) with data = bytes, or with
data = None and a size (a hole: the file is written sparse, so a
Qwen3-4B-shaped file of several GB costs no disk).  `raw_header_hook` lets a
test corrupt the encoded header.
"""
from __future__ import annotations

import struct

import numpy as np

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
F32, F16, Q8_0, Q6_K = 0, 1, 8, 14

_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
# {type: (elements per block, bytes per block)} for the types the tests write
TYPE_SIZE = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q6_K: (256, 210)}


def gguf_string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def encode_value(vtype: int, value) -> bytes:
    """A value without its type tag.  ARRAY values are (element_type, [items])."""
    if vtype == STRING:
        return gguf_string(value)
    if vtype == ARRAY:
        et, items = value
        return struct.pack("<IQ", et, len(items)) + b"".join(encode_value(et, v) for v in items)
    return struct.pack(_SCALAR[vtype], value)


def tensor_nbytes(dims, ttype) -> int:
    n = int(np.prod(dims, dtype=np.uint64)) if dims else 1
    bs, ts = TYPE_SIZE.get(ttype, (1, 4))
    return (n + bs - 1) // bs * ts


def align(x: int, a: int) -> int:
    return x + (a - x % a) % a


def write_gguf(path, metadata, tensors, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF",
               raw_header_hook=None, tail: bytes = b""):
    """metadata: [(key, vtype, value)]; tensors: [(name, dims, ttype, data_or_None[, size])].
    Returns {name: offset within the data region}."""
    out = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    for key, vtype, value in metadata:
        out += gguf_string(key) + struct.pack("<I", vtype) + encode_value(vtype, value)
    offsets, cur = {}, 0
    sizes = []
    for t in tensors:
        name, dims, ttype, data = t[:4]
        size = len(data) if data is not None else (t[4] if len(t) > 4 else tensor_nbytes(dims, ttype))
        sizes.append(size)
        offsets[name] = cur
        out += gguf_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ttype, cur)
        cur = align(cur + size, alignment)
    if raw_header_hook is not None:
        out = bytearray(raw_header_hook(bytes(out)))
    data_start = align(len(out), alignment)
    with open(path, "wb") as f:
        f.write(out)
        f.write(b"\0" * (data_start - len(out)))
        end = data_start
        for t, size in zip(tensors, sizes):
            name, data = t[0], t[3]
            at = data_start + offsets[name]
            if data is not None:
                f.seek(at)
                f.write(data)
            end = max(end, at + size)
        f.seek(end)
        f.write(tail)
        f.truncate(end + len(tail))
    return offsets
