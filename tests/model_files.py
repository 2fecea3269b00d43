"""Synthetic Qwen3 GGUF files and the oracle's forward over them (test
infrastructure).

write_tiny_qwen3 writes a small model with random weights in the tensor
layout the reference loads (src/model/qwen3.cu:190-223): token_embd Q8_0
[embed, vocab] (tied LM head), output_norm F32, and per layer F32 norms,
optional F32 q/k/v biases and QK-norm weights, and Q6_K projections.

oracle_forward runs the reference's forward (src/model/qwen3.cu:240-341)
launcher by launcher on the CPU oracle, for tokens at positions 0, 1, ...
"""
from __future__ import annotations

import numpy as np

from gguf_writer import F32, FLOAT32, Q6_K, Q8_0, STRING, UINT32, write_gguf
from oracle_py import make_q6k_matrix, make_q8_0_table

TINY = dict(n_layers=2, embed=512, ff=768, n_heads=4, n_kv=2, head_dim=128, vocab=1024)
TOKENS = [5, 1023, 0, 77, 512, 5, 9, 300]
# End-to-end bar on logits, per position: max|got - oracle| <= E2E_TOL *
# max|oracle|.  Moving every op's fp32 output by one unit in the last place
# moves these logits by up to ~6e-4 of max|logit| (the binary16 conversions
# before each projection turn rare one-ulp differences into 2^-11 steps);
# tests/test_oracle_forward.py checks the bar stays above that noise.
E2E_TOL = 4e-3


def write_tiny_qwen3(path, seed=0, *, arch="qwen3", qk_norm=True, bias=False, keys=True, alignment=32,
                     rope=1e6, eps=1e-6, **dims):
    d = dict(TINY, **dims)
    rng = np.random.default_rng(seed)
    E, FF, NH, NKV, HD, V = d["embed"], d["ff"], d["n_heads"], d["n_kv"], d["head_dim"], d["vocab"]
    Q, KV = NH * HD, NKV * HD
    norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
    t = {"token_embd.weight": ([E, V], Q8_0, make_q8_0_table(rng, V, E)),
         "output_norm.weight": ([E], F32, norm(E))}
    for l in range(d["n_layers"]):
        p = f"blk.{l}."
        t[p + "attn_norm.weight"] = ([E], F32, norm(E))
        t[p + "attn_q.weight"] = ([E, Q], Q6_K, make_q6k_matrix(rng, Q, E))
        t[p + "attn_k.weight"] = ([E, KV], Q6_K, make_q6k_matrix(rng, KV, E))
        t[p + "attn_v.weight"] = ([E, KV], Q6_K, make_q6k_matrix(rng, KV, E))
        if bias:
            t[p + "attn_q.bias"] = ([Q], F32, rng.standard_normal(Q).astype(np.float32))
            t[p + "attn_k.bias"] = ([KV], F32, rng.standard_normal(KV).astype(np.float32))
            t[p + "attn_v.bias"] = ([KV], F32, rng.standard_normal(KV).astype(np.float32))
        if qk_norm:
            t[p + "attn_q_norm.weight"] = ([HD], F32, norm(HD))
            t[p + "attn_k_norm.weight"] = ([HD], F32, norm(HD))
        t[p + "attn_output.weight"] = ([Q, E], Q6_K, make_q6k_matrix(rng, E, Q))
        t[p + "ffn_norm.weight"] = ([E], F32, norm(E))
        t[p + "ffn_gate.weight"] = ([E, FF], Q6_K, make_q6k_matrix(rng, FF, E))
        t[p + "ffn_up.weight"] = ([E, FF], Q6_K, make_q6k_matrix(rng, FF, E))
        t[p + "ffn_down.weight"] = ([FF, E], Q6_K, make_q6k_matrix(rng, E, FF))
    meta = [("general.architecture", STRING, arch),
            (f"{arch}.block_count", UINT32, d["n_layers"]),
            (f"{arch}.embedding_length", UINT32, E),
            (f"{arch}.feed_forward_length", UINT32, FF),
            (f"{arch}.attention.head_count", UINT32, NH),
            (f"{arch}.attention.head_count_kv", UINT32, NKV)]
    if keys:
        meta += [(f"{arch}.attention.key_length", UINT32, HD),
                 (f"{arch}.rope.freq_base", FLOAT32, rope),
                 (f"{arch}.attention.layer_norm_rms_epsilon", FLOAT32, eps)]
    if alignment != 32:
        meta.append(("general.alignment", UINT32, alignment))
    write_gguf(path, meta, [(n, dims_, tt, np.ascontiguousarray(a).tobytes()) for n, (dims_, tt, a) in t.items()],
               alignment=alignment)
    cfg = dict(d, rope=rope if keys else 10000.0, eps=eps if keys else 1e-5, qk_norm=qk_norm, bias=bias)
    if not keys:
        cfg["head_dim"] = E // NH  # the reference's fallback, src/model/qwen3.cu:152-157
    return {n: a for n, (_, _, a) in t.items()}, cfg


def oracle_forward(o, W, cfg, tokens, max_ctx):
    """Logits [len(tokens), vocab] for tokens at positions 0..; KV caches kept
    as binary16 [max_ctx, kv_dim] per layer, as the reference's."""
    E, FF, NH, NKV, HD, V = cfg["embed"], cfg["ff"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["vocab"]
    eps, base = cfg["eps"], cfg["rope"]
    kc = [np.zeros((max_ctx, NKV * HD), np.uint16) for _ in range(cfg["n_layers"])]
    vc = [np.zeros((max_ctx, NKV * HD), np.uint16) for _ in range(cfg["n_layers"])]
    table = W["token_embd.weight"]
    out = []
    for pos, tok in enumerate(tokens):
        h = o.embed_q8_0(table, tok, E)
        for l in range(cfg["n_layers"]):
            p = f"blk.{l}."
            g = lambda n: W.get(p + n)  # noqa: E731
            residual = h.copy()
            x16 = o.f32_to_f16(o.rms_norm(h, g("attn_norm.weight"), eps))
            q = o.gemv_q6k(g("attn_q.weight"), x16, g("attn_q.bias"))
            k = o.gemv_q6k(g("attn_k.weight"), x16, g("attn_k.bias"))
            v = o.gemv_q6k(g("attn_v.weight"), x16, g("attn_v.bias"))
            q, k = q.reshape(NH, HD), k.reshape(NKV, HD)
            if g("attn_q_norm.weight") is not None and g("attn_k_norm.weight") is not None:
                q = o.rms_norm_per_head(q, g("attn_q_norm.weight"), eps)
                k = o.rms_norm_per_head(k, g("attn_k_norm.weight"), eps)
            q, k = o.apply_rope(q, k, pos, base)
            kc[l], vc[l] = o.store_kv(kc[l], vc[l], k.reshape(-1), v, pos)
            att = o.gqa_attention(q.reshape(-1), kc[l], vc[l], NH, NKV, HD, pos + 1)
            h = o.residual_add(o.gemv_q6k(g("attn_output.weight"), o.f32_to_f16(att)), residual)
            residual = h.copy()
            x16 = o.f32_to_f16(o.rms_norm(h, g("ffn_norm.weight"), eps))
            act = o.silu_mul(o.gemv_q6k(g("ffn_gate.weight"), x16), o.gemv_q6k(g("ffn_up.weight"), x16))
            h = o.residual_add(o.gemv_q6k(g("ffn_down.weight"), o.f32_to_f16(act)), residual)
        h = o.rms_norm_inplace(h, W["output_norm.weight"], eps)
        out.append(o.gemv_q8_0(table, h))
    return np.stack(out), kc, vc
