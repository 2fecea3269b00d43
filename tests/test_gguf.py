"""The GGUF reader (include/fence/gguf.h) on synthetic files; no GPU needed.

test_reference_checks_* repeats the reference's own parser test
(tests/test_gguf_parser.cpp:60-199, which needs the real Qwen3-4B file) on a
file of the same shape written here: 398 tensors with Qwen3-4B's names, dims
and types, the same metadata, a tokenizer array to skip, and holes for the
tensor data (sparse, so the >3 GB file costs no disk).  The other tests pin
the format rules the reference's parser implements and the malformed-file
checks this reader adds.
"""
import ctypes
import struct

import numpy as np
import pytest

import fence_model as M
from fence_ops import FenceError
from gguf_writer import (ARRAY, BOOL, F32, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, Q6_K, Q8_0, STRING,
                         UINT8, UINT16, UINT32, UINT64, align, tensor_nbytes, write_gguf)

E, FF, NQ, NKV, HD, V, L = 2560, 9728, 32, 8, 128, 151936, 36


def qwen3_4b_tensors():
    t = [("output_norm.weight", [E], F32), ("token_embd.weight", [E, V], Q8_0)]
    for l in range(L):
        p = f"blk.{l}."
        t += [(p + "attn_norm.weight", [E], F32), (p + "attn_q.weight", [E, NQ * HD], Q6_K),
              (p + "attn_k.weight", [E, NKV * HD], Q6_K), (p + "attn_v.weight", [E, NKV * HD], Q6_K),
              (p + "attn_q_norm.weight", [HD], F32), (p + "attn_k_norm.weight", [HD], F32),
              (p + "attn_output.weight", [NQ * HD, E], Q6_K), (p + "ffn_norm.weight", [E], F32),
              (p + "ffn_gate.weight", [E, FF], Q6_K), (p + "ffn_up.weight", [E, FF], Q6_K),
              (p + "ffn_down.weight", [FF, E], Q6_K)]
    return t


QWEN3_4B_META = [
    ("general.architecture", STRING, "qwen3"),
    ("general.name", STRING, "synthetic Qwen3-4B layout"),
    ("qwen3.block_count", UINT32, L),
    ("qwen3.context_length", UINT32, 262144),
    ("qwen3.embedding_length", UINT32, E),
    ("qwen3.feed_forward_length", UINT32, FF),
    ("qwen3.attention.head_count", UINT32, NQ),
    ("qwen3.attention.head_count_kv", UINT32, NKV),
    ("qwen3.rope.freq_base", FLOAT32, 5000000.0),
    ("qwen3.attention.layer_norm_rms_epsilon", FLOAT32, 1e-6),
    ("qwen3.attention.key_length", UINT32, HD),
    ("qwen3.attention.value_length", UINT32, HD),
    ("tokenizer.ggml.model", STRING, "gpt2"),
    ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"tok{i}" for i in range(3000)])),
    ("tokenizer.ggml.token_type", ARRAY, (INT32, list(range(3000)))),
    ("tokenizer.ggml.merges", ARRAY, (STRING, ["a b", "c d"])),
    ("tokenizer.ggml.eos_token_id", UINT32, 151645),
    ("general.file_type", UINT32, 18),
]


@pytest.fixture(scope="module")
def qwen3_4b_file(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf") / "qwen3-4b-layout.gguf"
    norm = (1.0 + 0.01 * np.arange(E, dtype=np.float32)).tobytes()
    q_head = bytes(range(1, 17))  # non-zero first bytes of blk.0.attn_q.weight
    tensors = []
    for name, dims, tt in qwen3_4b_tensors():
        if name == "output_norm.weight":
            tensors.append((name, dims, tt, norm))
        elif name == "blk.0.attn_q.weight":
            tensors.append((name, dims, tt, q_head + b"\0" * (tensor_nbytes(dims, tt) - 16)))
        else:
            tensors.append((name, dims, tt, None))
    write_gguf(path, QWEN3_4B_META, tensors)
    return path


def test_reference_checks_header_and_metadata(qwen3_4b_file):
    """tests/test_gguf_parser.cpp:69-107"""
    with M.GGUF(qwen3_4b_file) as g:
        assert g.version == 3
        assert g.tensor_count == 398
        assert g.file_size > 3_000_000_000
        assert g.get_string("general.architecture") == "qwen3"
        assert g.get_u32("qwen3.block_count") == 36
        assert g.get_u32("qwen3.embedding_length") == 2560
        assert g.get_u32("qwen3.feed_forward_length") == 9728
        assert g.get_u32("qwen3.attention.head_count") == 32
        assert g.get_u32("qwen3.attention.head_count_kv") == 8
        assert g.get_u32("qwen3.attention.key_length") == 128
        assert abs(g.get_f32("qwen3.attention.layer_norm_rms_epsilon") - 1e-6) < 1e-8
        assert g.get_f32("qwen3.rope.freq_base") > 4e6


def test_reference_checks_tensors(qwen3_4b_file):
    """tests/test_gguf_parser.cpp:110-176"""
    with M.GGUF(qwen3_4b_file) as g:
        t = g.find_tensor("output_norm.weight")
        assert t and t["n_dims"] == 1 and t["dims"][0] == 2560 and t["type"] == M.F32
        assert t["data"] and t["data_size_bytes"] == 2560 * 4
        t = g.find_tensor("token_embd.weight")
        assert t and t["n_dims"] == 2 and t["dims"][:2] == (2560, 151936) and t["type"] == M.Q8_0 and t["data"]
        t = g.find_tensor("blk.0.attn_q.weight")
        assert t and t["n_dims"] == 2 and t["dims"][:2] == (2560, 4096) and t["type"] == M.Q6_K and t["data"]
        assert t["data_size_bytes"] == 2560 * 4096 // 256 * 210
        t = g.find_tensor("blk.0.attn_k.weight")
        assert t["dims"][:2] == (2560, 1024) and t["type"] == M.Q6_K
        assert g.find_tensor("blk.35.ffn_down.weight") is not None
        assert g.find_tensor("nonexistent.tensor") is None


def test_reference_checks_data_pointers(qwen3_4b_file):
    """tests/test_gguf_parser.cpp:179-193: the data pointers read the file's bytes."""
    with M.GGUF(qwen3_4b_file) as g:
        norm = np.frombuffer(g.tensor_bytes("output_norm.weight"), np.float32)
        assert norm[0] != 0 and np.array_equal(norm, 1.0 + 0.01 * np.arange(E, dtype=np.float32))
        assert g.tensor_bytes("blk.0.attn_q.weight")[:16] == bytes(range(1, 17))


def test_layout_offsets_sizes_and_order(qwen3_4b_file):
    with M.GGUF(qwen3_4b_file) as g:
        assert g.alignment == 32 and g.data_offset % 32 == 0
        prev_end = 0
        for i, (name, dims, tt) in enumerate(qwen3_4b_tensors()):
            t = g.tensor_at(i)
            assert t["name"] == name and t["offset"] % 32 == 0 and t["offset"] >= prev_end
            assert t["data_size_bytes"] == tensor_nbytes(dims, tt)
            assert t["dims"] == tuple(dims) + (1,) * (4 - len(dims))  # unused dims read as 1
            prev_end = t["offset"] + t["data_size_bytes"]
        assert g.data_offset + prev_end == g.file_size


def test_metadata_value_types_and_arrays(tmp_path):
    meta = [("u8", UINT8, 200), ("i8", INT8, -5), ("u16", UINT16, 60000), ("i16", INT16, -30000),
            ("u32", UINT32, 4000000000), ("i32", INT32, -2000000000), ("f32", FLOAT32, 1.5),
            ("b", BOOL, True), ("s", STRING, "héllo"), ("u64", UINT64, 2**60), ("i64", INT64, -2**60),
            ("f64", FLOAT64, 2.25), ("arr", ARRAY, (UINT16, [1, 2, 3])),
            ("nested", ARRAY, (ARRAY, [(STRING, ["x", "yz"]), (FLOAT64, [1.0])])),
            ("after", UINT32, 7)]
    p = tmp_path / "m.gguf"
    write_gguf(p, meta, [("t", [4], F32, np.ones(4, np.float32).tobytes())])
    with M.GGUF(p) as g:
        assert g.metadata_count == len(meta)
        for key, vt, _ in meta:
            assert g.metadata_type(key) == (None if vt == ARRAY else vt), key
        assert g.get_u32("u32") == 4000000000 and g.get_i32("i32") == -2000000000
        assert g.get_u64("u64") == 2**60 and g.get_f32("f32") == 1.5 and g.get_bool("b") is True
        assert g.get_string("s") == "héllo" and g.get_u32("after") == 7
        with pytest.raises(KeyError):
            g.get_u32("arr")  # arrays are skipped, not stored
        with pytest.raises(KeyError):
            g.get_u32("missing")
        with pytest.raises(TypeError):
            g.get_u32("i32")
        with pytest.raises(TypeError):
            g.get_string("u64")


def test_alignment_key(tmp_path):
    data = np.arange(8, dtype=np.float32).tobytes()
    for a in (64, 1, 0):
        p = tmp_path / f"a{a}.gguf"
        meta = [("general.alignment", UINT32, a), ("pad", STRING, "x" * 3)]
        eff = a if a else 32  # 0 is ignored and the default 32 stays
        write_gguf(p, meta, [("t0", [3], F32, data[:12]), ("t1", [8], F32, data)], alignment=eff)
        with M.GGUF(p) as g:
            assert g.alignment == eff and g.data_offset % eff == 0
            assert g.find_tensor("t1")["offset"] == align(12, eff)
            assert g.tensor_bytes("t1") == data


def test_version_2_is_read(tmp_path):
    p = tmp_path / "v2.gguf"
    write_gguf(p, [("k", UINT32, 1)], [("t", [2], F32, b"\1" * 8)], version=2)
    with M.GGUF(p) as g:
        assert g.version == 2 and g.get_u32("k") == 1


def test_unknown_tensor_type_is_sized_as_f32(tmp_path):
    """src/gguf/gguf_parser.cpp:47-49: an unknown type counts as {1, 4}."""
    p = tmp_path / "u.gguf"
    write_gguf(p, [], [("t", [5], 99, b"\0" * 20)])
    with M.GGUF(p) as g:
        assert g.find_tensor("t")["data_size_bytes"] == 20


def test_duplicate_names_resolve_to_the_last(tmp_path):
    p = tmp_path / "d.gguf"
    write_gguf(p, [("k", UINT32, 1), ("k", UINT32, 2)], [("t", [1], F32, b"\1" * 4), ("t", [2], F32, b"\2" * 8)])
    with M.GGUF(p) as g:
        assert g.get_u32("k") == 2 and g.find_tensor("t")["dims"][0] == 2


def _bad(path):
    with pytest.raises(FenceError) as e:
        M.GGUF(path)
    assert e.value.status == M.BAD_FILE
    return e.value.reason


def test_rejects_bad_magic_version_and_missing_files(tmp_path):
    p = tmp_path / "x.gguf"
    write_gguf(p, [], [], magic=b"GGML")
    assert "magic" in _bad(p)
    for v in (1, 4):
        write_gguf(p, [], [], version=v)
        assert "version" in _bad(p)
    assert "cannot open" in _bad(tmp_path / "absent.gguf")
    (tmp_path / "empty.gguf").write_bytes(b"")
    _bad(tmp_path / "empty.gguf")


def test_rejects_every_truncation(tmp_path):
    """Cut a valid file at every byte of its header: never read past the end."""
    p = tmp_path / "full.gguf"
    meta = [("s", STRING, "abc"), ("arr", ARRAY, (STRING, ["a", "bb"])), ("u", UINT32, 3)]
    write_gguf(p, meta, [("t", [4], F32, np.ones(4, np.float32).tobytes())])
    full = p.read_bytes()
    with M.GGUF(p) as g:
        header_end = g.data_offset
    cut = tmp_path / "cut.gguf"
    for n in range(1, header_end):
        cut.write_bytes(full[:n])
        _bad(cut)


def test_rejects_malformed_tensor_infos(tmp_path):
    p = tmp_path / "m.gguf"
    write_gguf(p, [], [("t", [1, 1, 1, 1, 1], F32, b"\0" * 4)])
    assert "dims" in _bad(p)
    # data offset beyond the file (src/gguf/gguf_parser.cpp:329-335)
    write_gguf(p, [], [("t", [4], F32, b"\0" * 16)],
               raw_header_hook=lambda h: h[:-8] + struct.pack("<Q", 1 << 20))
    assert "exceeds file size" in _bad(p)
    # data running past the end: rejected here (the reference checks the first byte only)
    write_gguf(p, [], [("t", [1000], F32, b"\0" * 16)])
    assert "past the end" in _bad(p)
    # dims whose product wraps 128 bits to 0 (2^43 * 2^43 * 2^42 = 2^128): caught before the wrap
    write_gguf(p, [], [("t", [1 << 43, 1 << 43, 1 << 42], F32, b"\0" * 16)])
    assert "more elements than the file" in _bad(p)
    write_gguf(p, [], [("t", [1 << 40, 1 << 40], Q8_0, b"\0" * 34)])
    assert "more elements than the file" in _bad(p)


def test_rejects_counts_and_lengths_beyond_the_file(tmp_path):
    p = tmp_path / "c.gguf"
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 1 << 60, 0))
    assert "tensor count" in _bad(p)
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1 << 60))
    assert "metadata count" in _bad(p)
    # a string claiming 2^63 bytes
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 63) + b"k" * 16)
    assert "end of file" in _bad(p)
    # an array of 2^62 u32
    body = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", ARRAY,
                                                                                               UINT32, 1 << 62)
    p.write_bytes(body + b"\0" * 16)
    assert "end of file" in _bad(p)
    # an unknown value type
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
                  + b"\0" * 16)
    assert "type" in _bad(p)


def test_rejects_deeply_nested_arrays(tmp_path):
    value = (UINT8, [1])
    for _ in range(20):
        value = (ARRAY, [value])
    p = tmp_path / "n.gguf"
    write_gguf(p, [("deep", ARRAY, value)], [])
    assert "nested" in _bad(p)
    value = (UINT8, [1])
    for _ in range(10):
        value = (ARRAY, [value])
    write_gguf(p, [("deep", ARRAY, value), ("k", UINT32, 5)], [])
    with M.GGUF(p) as g:
        assert g.get_u32("k") == 5


def test_random_corruptions_never_read_out_of_bounds(tmp_path):
    """Flip, overwrite or cut random bytes of a valid file's header 400 times:
    every open either succeeds (and every tensor's data lies inside the file)
    or fails cleanly with BAD_FILE -- never a crash or an out-of-file read."""
    rng = np.random.default_rng(2024)
    p = tmp_path / "ok.gguf"
    meta = [("general.architecture", STRING, "qwen3"), ("qwen3.block_count", UINT32, 2),
            ("tok", ARRAY, (STRING, ["a", "bc", "def"])), ("f", FLOAT32, 0.5), ("n", ARRAY, (INT32, [1, 2, 3]))]
    tensors = [("a", [64], F32, np.arange(64, dtype=np.float32).tobytes()),
               ("b", [256, 2], Q6_K, bytes(2 * 210)), ("c", [32, 3], Q8_0, bytes(3 * 34))]
    write_gguf(p, meta, tensors)
    good = bytearray(p.read_bytes())
    with M.GGUF(p) as g:
        header = g.data_offset
    bad = tmp_path / "bad.gguf"
    opened = 0
    for trial in range(400):
        b = bytearray(good)
        kind = trial % 3
        if kind == 0:  # flip bits in a few header bytes
            for i in rng.integers(0, header, size=int(rng.integers(1, 4))):
                b[i] ^= int(rng.integers(1, 256))
        elif kind == 1:  # overwrite a little-endian u64 with something large
            i = int(rng.integers(0, header - 8))
            big = [2**63, 2**40, 2**32 - 1, 1 << 20, 2**64 - 1][int(rng.integers(0, 5))]
            b[i:i + 8] = big.to_bytes(8, "little")
        else:  # truncate
            b = b[:int(rng.integers(1, len(b)))]
        bad.write_bytes(bytes(b))
        try:
            g = M.GGUF(bad)
        except FenceError as e:
            assert e.status == M.BAD_FILE
            continue
        with g:
            opened += 1
            for i in range(g.tensor_count):
                t = g.tensor_at(i)
                assert g.data_offset + t["offset"] + t["data_size_bytes"] <= g.file_size
                assert t["n_dims"] <= 4
                if t["data_size_bytes"]:  # the data is readable: touch its last byte
                    ctypes.string_at(t["data"] + t["data_size_bytes"] - 1, 1)
    assert opened > 0  # some mutations land in string bytes and keep the file valid
