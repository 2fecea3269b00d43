"""Model-file checks of fence_model_load that fail before any device work
(no GPU needed): unreadable files, and tensors that are missing or of the
wrong type or shape for the forward (the reference would copy a null pointer
or misread the data, src/model/qwen3.cu:99-105,190-223)."""
import numpy as np
import pytest

import fence_model as M
from fence_ops import EINVAL, FenceError
from gguf_writer import F32, FLOAT32, Q6_K, STRING, UINT32, write_gguf
from model_files import write_tiny_qwen3


def load_error(path, max_ctx=16):
    with pytest.raises(FenceError) as e:
        M.Model(path, max_ctx=max_ctx)
    return e.value.status, e.value.reason


def rewrite(src, dst, drop=(), replace=None):
    """Copy a GGUF file with tensors dropped or replaced (name -> (dims, type, bytes))."""
    with M.GGUF(src) as g:
        meta = []
        for key in ("general.architecture",):
            meta.append((key, STRING, g.get_string(key)))
        arch = meta[0][2]
        for k in ("block_count", "embedding_length", "feed_forward_length", "attention.head_count",
                  "attention.head_count_kv", "attention.key_length"):
            meta.append((f"{arch}.{k}", UINT32, g.get_u32(f"{arch}.{k}")))
        for k in ("rope.freq_base", "attention.layer_norm_rms_epsilon"):
            meta.append((f"{arch}.{k}", FLOAT32, g.get_f32(f"{arch}.{k}")))
        tensors = []
        for i in range(g.tensor_count):
            t = g.tensor_at(i)
            if t["name"] in drop:
                continue
            if replace and t["name"] in replace:
                dims, tt, data = replace[t["name"]]
                tensors.append((t["name"], dims, tt, data))
            else:
                tensors.append((t["name"], list(t["dims"][:t["n_dims"]]), t["type"], g.tensor_bytes(t["name"])))
    write_gguf(dst, meta, tensors)


@pytest.fixture(scope="module")
def good(tmp_path_factory):
    p = tmp_path_factory.mktemp("load") / "good.gguf"
    write_tiny_qwen3(p, seed=5)
    return p


def test_unreadable_files(tmp_path):
    st, why = load_error(tmp_path / "absent.gguf")
    assert st == M.BAD_FILE and "cannot open" in why
    (tmp_path / "junk.gguf").write_bytes(b"not a gguf file at all" * 4)
    st, why = load_error(tmp_path / "junk.gguf")
    assert st == M.BAD_FILE and "magic" in why


def test_missing_required_tensor(good, tmp_path):
    for name in ("token_embd.weight", "output_norm.weight", "blk.1.ffn_down.weight", "blk.0.attn_norm.weight"):
        p = tmp_path / "m.gguf"
        rewrite(good, p, drop={name})
        st, why = load_error(p)
        assert st == M.UNSUPPORTED and name in why


def test_wrong_type_or_shape(good, tmp_path):
    p = tmp_path / "t.gguf"
    rewrite(good, p, replace={"blk.0.attn_q.weight": ([512, 512], F32, np.zeros(512 * 512, np.float32).tobytes())})
    st, why = load_error(p)
    assert st == M.UNSUPPORTED and "attn_q.weight is F32" in why
    rewrite(good, p, replace={"blk.1.ffn_up.weight": ([512, 512], Q6_K, bytes(512 * 2 * 210))})
    st, why = load_error(p)
    assert st == M.UNSUPPORTED and "shape" in why
    rewrite(good, p, replace={"blk.0.attn_q_norm.weight": ([64], F32, bytes(256))})
    st, why = load_error(p)
    assert st == M.UNSUPPORTED and "attn_q_norm" in why


def test_dimensions_the_kernels_cannot_run(tmp_path):
    p = tmp_path / "d.gguf"
    write_tiny_qwen3(p, seed=6, embed=320)  # Q6_K rows need K % 256 == 0
    st, why = load_error(p)
    assert st == M.UNSUPPORTED and "multiples of 256" in why


def test_missing_required_metadata(tmp_path):
    p = tmp_path / "k.gguf"
    write_gguf(p, [("general.architecture", STRING, "qwen3")], [("token_embd.weight", [32, 4], 8, bytes(4 * 34))])
    st, why = load_error(p)
    assert st == M.UNSUPPORTED and "block_count" in why


def test_bad_arguments(good):
    with pytest.raises(FenceError) as e:
        M.Model(good, max_ctx=0)
    assert e.value.status == EINVAL
