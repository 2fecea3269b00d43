"""A minimal GGUF writer: model files in the layout the reference's parser
reads (src/gguf/gguf_parser.cpp:144-345) -- header, metadata key/values,
tensor infos, then the tensor data region at the next multiple of the
alignment, each tensor at an aligned offset within it.  Used to write
synthetic models for the tests and the benchmark.

Tensors given as (name, dims, type, data) with data = bytes (or any object
with the buffer protocol), as (name, dims, type, fn, size) with fn() giving
the bytes when the tensor is written (so a large model never sits in host
memory whole), or with data = None and a size (a hole: the file is written
sparse, so a Qwen3-4B-shaped file of several GB costs no disk).
`raw_header_hook` lets a test corrupt the encoded header.
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
        if data is not None and not callable(data):
            size = memoryview(data).nbytes
        else:
            size = t[4] if len(t) > 4 else tensor_nbytes(dims, ttype)
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
                f.write(memoryview(data() if callable(data) else data).cast("B"))
            end = max(end, at + size)
        f.seek(end)
        f.write(tail)
        f.truncate(end + len(tail))
    return offsets


def synthetic_qwen3(path, seed=0, n_layers=36, embed=2560, ff=9728, n_heads=32, n_kv=8, head_dim=128,
                    vocab=151936, rope=5e6, eps=1e-6):
    """A Qwen3 model file of the given shape with random weights (defaults:
    Qwen3-4B, src/model/qwen3.h:19-44): Q8_0 token_embd (also the LM head),
    Q6_K projections, F32 norms.  Q6_K blocks have uniform random quants,
    sub-block scales uniform in [-8, 7] and d = 2^-10; Q8_0 blocks uniform
    int8 with d = 2^-12; norm weights 1 + N(0, 0.1).  The random bytes come
    from a 64 MiB pool read from a random offset per tensor, so a multi-GB
    model is written in seconds.  Returns the byte size of the tensor data."""
    rng = np.random.default_rng(seed)
    pool = rng.integers(0, 2**63, size=(64 << 20) // 8, dtype=np.uint64).view(np.uint8)
    scratch = np.empty(0, np.uint8)  # reused for every quantized tensor

    def rand_bytes(n):
        nonlocal scratch
        if scratch.size < n:
            scratch = np.empty(n, np.uint8)
        out, off, done = scratch[:n], int(rng.integers(0, pool.size)), 0
        while done < n:
            take = min(n - done, pool.size - off)
            out[done:done + take] = pool[off:off + take]
            done, off = done + take, 0
        return out

    def q6k(m, k):
        def make():
            a = rand_bytes(m * (k // 256) * 210).reshape(-1, 210)
            a[:, 192:208] &= 15
            a[:, 192:208] += np.uint8(248)  # int8 scales -8..7
            a[:, 208], a[:, 209] = 0x00, 0x14  # d = binary16 2^-10
            return a
        return make, m * (k // 256) * 210

    def norm(n):
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    def table():
        t = rand_bytes(vocab * (embed // 32) * 34).reshape(-1, 34)
        t[:, 0], t[:, 1] = 0x00, 0x0C  # d = binary16 2^-12
        return t

    q, kv = n_heads * head_dim, n_kv * head_dim
    tensors = [("token_embd.weight", [embed, vocab], Q8_0, table, vocab * (embed // 32) * 34),
               ("output_norm.weight", [embed], F32, norm(embed))]
    for l in range(n_layers):
        p = f"blk.{l}."
        tensors += [(p + "attn_norm.weight", [embed], F32, norm(embed)),
                    (p + "attn_q.weight", [embed, q], Q6_K, *q6k(q, embed)),
                    (p + "attn_k.weight", [embed, kv], Q6_K, *q6k(kv, embed)),
                    (p + "attn_v.weight", [embed, kv], Q6_K, *q6k(kv, embed)),
                    (p + "attn_q_norm.weight", [head_dim], F32, norm(head_dim)),
                    (p + "attn_k_norm.weight", [head_dim], F32, norm(head_dim)),
                    (p + "attn_output.weight", [q, embed], Q6_K, *q6k(embed, q)),
                    (p + "ffn_norm.weight", [embed], F32, norm(embed)),
                    (p + "ffn_gate.weight", [embed, ff], Q6_K, *q6k(ff, embed)),
                    (p + "ffn_up.weight", [embed, ff], Q6_K, *q6k(ff, embed)),
                    (p + "ffn_down.weight", [ff, embed], Q6_K, *q6k(embed, ff))]
    arch = "qwen3"
    meta = [("general.architecture", STRING, arch), (f"{arch}.block_count", UINT32, n_layers),
            (f"{arch}.embedding_length", UINT32, embed), (f"{arch}.feed_forward_length", UINT32, ff),
            (f"{arch}.attention.head_count", UINT32, n_heads), (f"{arch}.attention.head_count_kv", UINT32, n_kv),
            (f"{arch}.attention.key_length", UINT32, head_dim), (f"{arch}.rope.freq_base", FLOAT32, rope),
            (f"{arch}.attention.layer_norm_rms_epsilon", FLOAT32, eps)]
    write_gguf(path, meta, tensors)
    return sum(t[4] if len(t) > 4 else t[3].nbytes for t in tensors)
