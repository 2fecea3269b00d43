"""Pins of the oracle's forward (tests/model_files.oracle_forward), the
checker of the model GPU tests; CPU only.

1. Its wiring: an independent float64 numpy forward of the same model
   (weights dequantised by q6k_dequant_numpy / q8_0_dequant_numpy, numpy's
   own binary16 rounding, the textbook formulas of each stage) agrees with it.
   A dropped residual, swapped gate/up, wrong head grouping or a RoPE on the
   wrong pairs moves the logits by O(1).
2. The end-to-end bar of the GPU tests: perturbing every op's fp32 output by
   one unit in the last place moves this model's logits by well under the
   bar -- so the bar sits above the model's own fp32 noise, and not so far
   above that a wrong stage could pass.
"""
import numpy as np
import pytest

from model_files import E2E_TOL, TOKENS, oracle_forward, write_tiny_qwen3
from oracle_py import q6k_dequant_numpy, q8_0_dequant_numpy

CTX = 16


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    return write_tiny_qwen3(tmp_path_factory.mktemp("of") / "m.gguf", seed=1)


def numpy_forward(W, cfg, tokens):
    E, NH, NKV, HD, V = cfg["embed"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["vocab"]
    eps, base = cfg["eps"], cfg["rope"]
    f16 = lambda x: np.asarray(x, np.float64).astype(np.float16).astype(np.float64)  # noqa: E731
    norm = lambda x, w: x / np.sqrt(np.mean(x * x) + eps) * w  # noqa: E731
    table = q8_0_dequant_numpy(W["token_embd.weight"], np.arange(V), E).astype(np.float64)
    deq = {n: q6k_dequant_numpy(a, a.shape[1] // 210 * 256) for n, a in W.items() if a.dtype == np.uint8
           and n != "token_embd.weight"}
    inv = base ** (-np.arange(0, HD, 2) / HD)

    def rope(x, pos):  # NeoX pairs (i, i + HD/2)
        a, b = x[:, :HD // 2], x[:, HD // 2:]
        c, s = np.cos(pos * inv), np.sin(pos * inv)
        return np.concatenate([a * c - b * s, a * s + b * c], axis=1)

    K = [np.zeros((0, NKV, HD)) for _ in range(cfg["n_layers"])]
    Vc = [np.zeros((0, NKV, HD)) for _ in range(cfg["n_layers"])]
    out = []
    for pos, tok in enumerate(tokens):
        h = table[tok].copy()
        for l in range(cfg["n_layers"]):
            p = f"blk.{l}."
            w = lambda n: W[p + n].astype(np.float64)  # noqa: E731
            x = f16(norm(h, w("attn_norm.weight")))
            q, k, v = (deq[p + f"attn_{t}.weight"] @ x for t in "qkv")
            if cfg["bias"]:
                q, k, v = q + w("attn_q.bias"), k + w("attn_k.bias"), v + w("attn_v.bias")
            q, k, v = q.reshape(NH, HD), k.reshape(NKV, HD), v.reshape(NKV, HD)
            if cfg["qk_norm"]:
                q = np.stack([norm(r, w("attn_q_norm.weight")) for r in q])
                k = np.stack([norm(r, w("attn_k_norm.weight")) for r in k])
            q, k = rope(q, pos), rope(k, pos)
            K[l] = np.concatenate([K[l], f16(k)[None]])
            Vc[l] = np.concatenate([Vc[l], f16(v)[None]])
            att = np.empty((NH, HD))
            for hq in range(NH):
                g = hq // (NH // NKV)
                s = K[l][:, g] @ q[hq] / np.sqrt(HD)
                pr = np.exp(s - s.max())
                att[hq] = (pr / pr.sum()) @ Vc[l][:, g]
            h = h + deq[p + "attn_output.weight"] @ f16(att.reshape(-1))
            x = f16(norm(h, w("ffn_norm.weight")))
            gt, up = deq[p + "ffn_gate.weight"] @ x, deq[p + "ffn_up.weight"] @ x
            h = h + deq[p + "ffn_down.weight"] @ f16(gt / (1 + np.exp(-gt)) * up)
        out.append(table @ norm(h, W["output_norm.weight"].astype(np.float64)))
    return np.stack(out)


def rel_err(a, b):
    return max(np.max(np.abs(a[p] - b[p])) / np.max(np.abs(b[p])) for p in range(b.shape[0]))


@pytest.mark.parametrize("variant", ["qwen3", "qwen2-style"])
def test_oracle_forward_matches_independent_numpy_forward(oracle, tmp_path, variant):
    if variant == "qwen3":
        W, cfg = write_tiny_qwen3(tmp_path / "a.gguf", seed=1)
    else:
        W, cfg = write_tiny_qwen3(tmp_path / "b.gguf", seed=2, qk_norm=False, bias=True, keys=False)
    ref, _, _ = oracle_forward(oracle, W, cfg, TOKENS[:6], CTX)
    ind = numpy_forward(W, cfg, TOKENS[:6])
    assert rel_err(ref, ind) <= E2E_TOL


class _Jitter:
    """Each call of the wrapped ops returns its fp32 outputs moved by -1, 0 or
    +1 unit in the last place at random."""

    def __init__(self, o, rng):
        self.o, self.rng = o, rng

    def __getattr__(self, name):
        f = getattr(self.o, name)
        if name in ("f32_to_f16", "store_kv", "embed_q8_0"):
            return f

        def one(x):
            if not (isinstance(x, np.ndarray) and x.dtype == np.float32):
                return x
            step = self.rng.integers(-1, 2, x.shape)
            up, down = np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf))
            return np.where(step > 0, up, np.where(step < 0, down, x)).astype(np.float32)

        def jittered(*a, **k):
            r = f(*a, **k)
            return tuple(one(x) for x in r) if isinstance(r, tuple) else one(r)
        return jittered


def test_end_to_end_bar_sits_above_fp32_noise(oracle, model):
    W, cfg = model
    ref, _, _ = oracle_forward(oracle, W, cfg, TOKENS, CTX)
    noise = max(rel_err(oracle_forward(_Jitter(oracle, np.random.default_rng(s)), W, cfg, TOKENS, CTX)[0], ref)
                for s in range(3))
    print(f"one-ulp noise moves the logits by {noise:.3g} of max|logit|")
    assert 0 < noise <= E2E_TOL / 2
